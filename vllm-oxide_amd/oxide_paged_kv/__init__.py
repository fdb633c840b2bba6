"""MI355X (gfx950) paged-KV hot path of vllm-oxide: Python front end.

The kernels live in liboxide_paged_kv.so (HIP, built in-tree by
vllm-oxide_amd/build.py); this package only binds them (ctypes) and generates
the synthetic workloads of the benchmark configurations.
"""
from ._lib import LIB_PATH, OxideError, load  # noqa: F401
from .ops import (CASCADE_MODES, DECODE_PATHS, build_decode_metadata, copy_blocks, decode_attn,  # noqa: F401
                  dtype_code, gather_blocks, shared_prefix_plan, shared_prefix_workspace_size,
                  prefill_attn, qk_norm_rope_and_cache, reshape_and_cache, rope_cos_sin_cache,
                  split_tokens, workspace_size)
