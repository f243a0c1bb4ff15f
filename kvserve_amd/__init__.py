"""kvserve_amd: MI355X-native (gfx950 / CDNA4) paged-attention backend for kvserve.

The attention hot path of kvserve (reshape_and_cache + paged attention) on hand-written
HIP kernels behind kvserve's attention-backend interface:

    from kvserve_amd import HipAttention, AttentionMetadata
    HipAttention.write_kv(k_cache, v_cache, k, v, meta.slot_mapping)
    out = HipAttention.forward(q, k_cache, v_cache, meta, scale, out=None)

The kernels live in libkvhip.so (C ABI: include/kvhip.h), built in-tree by
`python -m kvserve_amd.build`. There is no CPU fallback.
"""

from kvserve_amd.attention import (
    AttentionMetadata,
    HipAttention,
    build_metadata,
    get_backend,
    hip_available,
    hip_eligible,
    last_launch_kernels,
)

__all__ = [
    "AttentionMetadata",
    "HipAttention",
    "build_metadata",
    "get_backend",
    "hip_available",
    "hip_eligible",
    "last_launch_kernels",
]
