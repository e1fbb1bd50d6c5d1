"""rec_amd — MI355X (gfx950) GQA decode attention over a quantized KV cache.

Drop-in for the quantized-KV attention path of rec's engine
(engine/src/rec_mlx/model.py:40-139,165-211): a quantize-on-append cache with
the reference's cache surface and ``quantized_attention_with_sinks`` with its
signature, and the bf16 ``KVStorage`` / ``FixedKVCache`` path
(engine/src/rec_mlx/cache.py:48-150) with its decode attention, and the
int4 group-64 GEMV of the decoder's projections
(engine/src/rec_mlx/kernels/megakernel.py:161-232), running hand-written HIP
kernels through the C ABI in ``include/rec_amd.h``.
"""

from ._lib import RecError, load as library  # noqa: F401
from .attention import attend, dequantize_kv, quantized_attention_with_sinks, scaled_dot_product_attention  # noqa: F401
from .cache import MixedQuantizedKVCache, QuantizedKV, QuantizedKVCache, to_logical  # noqa: F401
from .gemv import Q4Matrix, q4_gemv, q4_gemv_parts, quantized_matmul  # noqa: F401
from .kvstorage import FixedKVCache, FixedSlidingKVCache, KVStorage, make_cache  # noqa: F401

__version__ = "0.1.0"
