"""nexusquant_amd: MI355X-native (gfx950) post-prefill KV-cache compression.

Drop-in for the reference's hot path (jagmarques/nexusquant v0.5.0):

    from nexusquant_amd import compress_kv_cache, nexusquant_evict
    compress_kv_cache(past_key_values, mode="quant_only", rope_base=500000.0,
                      key_bits=3, value_bits=2)
    with nexusquant_evict(model, quality="high") as nq:
        model.generate(input_ids, max_new_tokens=100)

All compute runs in the hand-written HIP library nexusquant_amd/lib/libnqamd.so
(build: `python -m nexusquant_amd.build`); there is no CPU fallback.
"""

__version__ = "0.1.0"

from .hadamard import hadamard_matrix, next_power_of_2  # noqa: F401
from .huggingface import nexusquant_evict  # noqa: F401
from .ops import PackedCodes, quantize_tensors  # noqa: F401
from .pipeline import (NexusQuantEvict, NexusQuantEvictTruncate, NexusQuantQuantOnly,  # noqa: F401
                       compress_kv_cache)
