"""MI355X-native Qwen3.5 Gated DeltaNet layer (hand-written HIP for gfx950 behind a C ABI).

    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP, Qwen35GDNStackHIP, GatedDeltaRuleHIP

The compute lives in libgdn_hip.so (include/gdn.h); these classes mirror the reference's layer and
recurrence-op objects.  Build the library with `python -m linear_attention_op_amd.build`.
"""

from ._lib import GdnError, GdnValueError, LIB_PATH  # noqa: F401
from .gated_delta import GatedDeltaRuleHIP  # noqa: F401
from .gdn_layer import (Qwen35GatedDeltaNetHIP, linear, quantize_fp8, quantize_mxfp4, quantize_mxint8,  # noqa: F401
                        weights_from_hf)
from .gdn_stack import Qwen35GDNStackHIP  # noqa: F401
from .checkpoint import linear_attention_layers, load_gdn_weights  # noqa: F401

__all__ = ["Qwen35GatedDeltaNetHIP", "Qwen35GDNStackHIP", "GatedDeltaRuleHIP", "linear", "quantize_fp8", "quantize_mxfp4",
           "quantize_mxint8", "weights_from_hf", "load_gdn_weights", "linear_attention_layers", "GdnError", "GdnValueError"]
