"""laii_amd -- MI355X (gfx950) attention path of the LFM2/LFM2.5/LFM3 engine.

The product is the native library laii_amd/liblfm_attn.so (C-ABI in
include/lfm_attn.h: HIP kernels + C11 host code).  This package is its Python
host mirror: ctypes bindings named after the reference's dispatch calls.
"""
from ._lib import LIB_PATH, LfmAttnError, load  # noqa: F401
from .attention import (  # noqa: F401
    GGML_IQ4_XS,
    GGML_Q4_0,
    GGML_Q4_K,
    GGML_Q5_K,
    GGML_Q6_K,
    GGML_Q8_0,
    CacheModel,
    DeviceArray,
    EngineContext,
    device_count,
    fnv1a64,
    gen1_gqa_step,
    gqa_f16_step,
    gqa_f16_varlen,
    gqa_f16_varlen_noalloc,
    gqa_heads,
    gqa_qkv_fused,
    kv_cache_shift_sinks,
    last_plan,
    lfm3_kv_cache_shift_sinks,
    lfm3_online_gqa_f16_dispatch,
    lfm3_prefill_f16,
    matmul_prequant,
    matmul_q4_K,
    online_gqa_f16,
    pointer_table,
    prefill_f16,
    qk_norm_rope,
    qkv_prologue,
    quantize_q8_K,
    require_gpu,
    rope_lut_lfm2,
    rope_lut_lfm3,
    rope_row_gen1,
    seg_plan,
    slot_of,
    store_fp32_to_fp16,
    sync,
)
