"""ctypes binding of ``libimie_gfx950.so`` (the gfx950 producer library).

The library is REQUIRED: ``lib()`` raises ``ImportError`` when the in-tree ``.so`` is missing, so no caller can
silently run without the HIP kernels. Whether a usable gfx950 device is present is a separate question answered
by ``device_available()`` (the reference's ``bonsai_gpu_available`` probe).
"""
from __future__ import annotations

import ctypes
from ctypes import c_int, c_int64, c_uint32, c_uint64, c_void_p
from functools import lru_cache
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libimie_gfx950.so"

# name -> (restype, argtypes). Every symbol declared in include/imie_bonsai.h and include/imie_nmc.h.
SIGNATURES = {
    # runtime (include/imie_bonsai.h)
    "bonsai_gpu_available": (c_int, []),
    "bonsai_gpu_mem_info": (c_int, [c_void_p, c_void_p]),
    "bonsai_gpu_abi_version": (c_int, []),
    "bonsai_gpu_last_error_code": (c_int, []),
    "bonsai_gpu_last_error": (ctypes.c_char_p, []),
    "imie_abi_version": (c_int, []),
    "imie_last_error": (ctypes.c_char_p, []),
    "imie_default_stream": (c_void_p, []),
    "imie_synchronize": (c_int, []),
    "imie_probe_mfma": (c_int, [c_void_p, c_void_p, c_void_p]),
    "imie_mfma_peak": (c_int, [c_void_p]),
    "imie_hbm_read_peak": (c_int, [c_int64, c_void_p]),
    "imie_sample_token": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "imie_sample_dev": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p]),
    "imie_sample_draw_probe": (c_int, [c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_logits_digest_dev": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_net_decode_sampled_dev": (c_int, [c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_int64, c_void_p, c_int64, c_int, c_void_p]),
    "imie_profile_begin": (None, []),
    "imie_profile_gemm_ops": (c_int, [c_void_p, c_int]),
    "imie_profile_read": (c_int, [c_int, c_void_p, c_void_p]),
    "imie_profile_end": (None, []),
    # host re-execution (receipt verifier)
    "imie_cpu_model_create": (c_int64, [c_int64] * 10 + [c_void_p] * 10 + [c_int64]),
    "imie_cpu_model_free": (None, [c_int64]),
    "imie_cpu_set_threads": (None, [c_int]),
    "imie_cpu_forward": (c_int, [c_int64, c_void_p, c_int64, c_int, c_void_p]),
    "imie_cpu_sample_token": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    # Q1_0 linear
    "bonsai_q1_linear_gpu": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "bonsai_q1_register_weight": (c_int64, [c_void_p, c_void_p, c_int64, c_int64]),
    "bonsai_q1_register_weight_i32": (c_int64, [c_void_p, c_void_p, c_int64, c_int64]),
    "bonsai_q1_register_weight_i32_gpu_layout": (c_int64, [c_void_p, c_void_p, c_int64, c_int64]),
    "bonsai_q1_register_weight_i32_bmma": (c_int64, [c_void_p, c_void_p, c_int64, c_int64]),
    "bonsai_q1_linear_dp4a_gpu": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int,
                                          c_void_p]),
    "bonsai_q1_apply_resident": (c_int, [c_int64, c_void_p, c_int64, c_int64, c_void_p]),
    "bonsai_q1_free_weights": (None, []),
    "bonsai_q1_resident_weight_bytes": (c_uint64, []),
    "imie_q1_repack_host": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "imie_q1_apply_dev": (c_int, [c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_q1_apply_dev_noalloc": (c_int, [c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_q1_weight_info": (c_int, [c_int64, c_void_p, c_void_p, c_void_p]),
    "imie_q1_linear_simple_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                          c_void_p, c_void_p]),
    # RMSNorm / element-wise
    "bonsai_rmsnorm_gpu": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_rmsnorm_fused_gpu": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_rmsnorm_dev": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                 c_void_p]),
    "bonsai_silu_gpu": (c_int, [c_void_p, c_int64, c_int64, c_void_p]),
    "imie_rope_neox_gpu": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
                                   c_int64, c_void_p]),
    "imie_argmax_gpu": (c_int, [c_void_p, c_int64, c_int64, c_void_p]),
    # attention
    "bonsai_attention_prefill_gpu": (c_int, [c_void_p] * 3 + [c_int64] * 8 + [c_void_p]),
    "bonsai_attention_decode_batched_gpu": (c_int, [c_void_p] * 4 + [c_int64] * 7 + [c_void_p]),
    "imie_attention_scores_probe": (c_int, [c_void_p] * 2 + [c_int64] * 8 + [c_void_p] * 2 + [c_int, c_void_p]),
    # resident model / decode context
    "bonsai_buf_upload_i64": (c_int64, [c_void_p, c_int64]),
    "imie_buf_device_ptr": (c_void_p, [c_int64]),
    "imie_buf_free_all": (None, []),
    "bonsai_prefill_forward_gpu": (c_int, [c_void_p] + [c_int64] * 10 + [c_void_p] * 11 + [c_int64] * 4
                                   + [c_void_p] * 3),
    "bonsai_decode_ctx_create": (c_int64, [c_int64] * 12 + [c_void_p] * 11 + [c_int64] * 4),
    "imie_net_create": (c_int64, [c_int64] * 11 + [c_void_p] * 11 + [c_int64] * 5 + [c_int]),
    "bonsai_decode_ctx_seed_seq": (c_int, [c_int64, c_int64, c_void_p, c_void_p, c_int64]),
    "bonsai_decode_step": (c_int, [c_int64, c_void_p, c_void_p, c_void_p]),
    "bonsai_decode_ctx_free": (None, [c_int64]),
    "imie_net_reset": (c_int, [c_int64]),
    "bonsai_gpu_reservation_create": (c_int64, [c_void_p, c_int64, c_void_p]),
    "bonsai_gpu_reservation_free": (None, [c_int64]),
    "imie_net_forward_dev": (c_int, [c_int64, c_void_p, c_void_p, c_int64, c_void_p]),
    "imie_net_head_dev": (c_int, [c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "imie_net_status": (c_int, [c_int64, c_int, c_void_p]),
    "imie_net_export_kv": (c_int, [c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "imie_embed_dev": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "imie_fx_isqrt_u128": (c_uint64, [c_uint64, c_uint64]),
    "imie_fx_recip_u64": (c_uint64, [c_uint64]),
    "imie_fx_isqrt_fast": (c_uint64, [c_uint64, c_uint64]),
    "imie_fx_norm_f64": (c_int, [c_int64, c_int, c_uint64, c_void_p]),
    "imie_silu_mul_host": (c_int64, [c_int64, c_int64, c_int64, c_int]),
    "imie_exp_clipped_host": (c_int64, [c_int64, c_int64, c_int]),
    "imie_prob_div_host": (c_int64, [c_int64, c_int64, c_uint64]),
    "imie_fx_div_u128": (c_uint64, [c_uint64, c_uint64, c_uint32]),
    "imie_net_set_caps": (c_int, [c_int64, c_void_p]),
    "imie_net_fill_kv": (c_int, [c_int64, c_uint64, c_void_p, c_void_p, c_int64, c_int64]),
    "imie_net_decode_dev": (c_int, [c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int,
                                    c_void_p]),
    # north-mini-code Q4_K / Q6_K (include/imie_nmc.h)
    "qk_cuda_abi_version": (c_int, []),
    "qk_cuda_available": (c_int, []),
    "qk_linear_cuda": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_int, c_void_p]),
    "qk_register_weight": (c_int64, [c_void_p, c_int64, c_int64, c_int]),
    "qk_resident_reserve": (c_int, [c_int64]),
    "qk_apply_resident": (c_int, [c_int64, c_void_p, c_int64, c_int, c_void_p]),
    "qk_apply_resident_grouped": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int, c_int64, c_void_p]),
    "qk_apply_resident_q4k_dp4a": (c_int, [c_int64, c_void_p, c_int64, c_int, c_int, c_void_p]),
    "qk_apply_resident_q6k_dp4a": (c_int, [c_int64, c_void_p, c_int64, c_int, c_int, c_void_p]),
    "qk_moe_ffn_batched": (c_int, [c_void_p] * 3 + [c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int,
                                                      c_void_p]),
    "qk_moe_ffn_batched_dp4a": (c_int, [c_void_p] * 3 + [c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_int,
                                                           c_int, c_void_p]),
    "qk_moe_ffn": (c_int, [c_void_p] * 3 + [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_void_p]),
    "qk_moe_ffn_dp4a": (c_int, [c_void_p] * 3 + [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_void_p]),
    "imie_moe_ffn_batched_dev": (c_int, [c_void_p] * 3 + [c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_int,
                                                            c_int, c_void_p, c_void_p]),
    "imie_moe_status": (c_int, [c_int, c_void_p]),
    "imie_fp16_fixed_probe": (c_int, [c_void_p, c_int64, c_int, c_void_p]),
    "qk_register_i64": (c_int64, [c_void_p, c_int64, c_int64]),
    "qk_rmsnorm_router": (c_int, [c_int64, c_int64, c_void_p, c_int64, c_int, c_int, c_uint64, c_int, c_int64, c_int64,
                                  c_void_p, c_void_p, c_void_p]),
    "qk_attention_bank_create": (c_int64, [c_int, c_int64, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "qk_attention_bank_import": (c_int, [c_int64, c_int, c_void_p, c_void_p, c_int64]),
    "qk_attention_bank_apply": (c_int, [c_int64, c_int, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int, c_int,
                                        c_int, c_int64, c_int64, c_void_p]),
    "qk_attention_bank_moe_configure": (c_int, [c_int64, c_int, c_int, c_int, c_int64, c_int64]),
    "qk_attention_bank_moe_bind": (c_int, [c_int64, c_int, c_int, c_int64, c_int64, c_int64]),
    "qk_attention_bank_moe_begin": (c_int, [c_int64, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                            c_void_p, c_int, c_int, c_uint64, c_int, c_int, c_int64, c_int, c_void_p,
                                            c_void_p]),
    "qk_attention_bank_moe_continue": (c_int, [c_int64, c_int, c_int, c_int, c_int64, c_void_p]),
    "qk_attention_bank_moe_export": (c_int, [c_int64, c_int64, c_void_p]),
    "qk_attention_bank_workspace_bytes": (c_uint64, [c_int64]),
    "qk_attention_bank_reset": (c_int, [c_int64]),
    "qk_attention_bank_destroy": (None, [c_int64]),
    "qk_free_all": (None, []),
    "qk_resident_count": (c_int64, []),
    "qk_resident_capacity": (c_int64, []),
    "qk_moe_workspace_allocations": (c_int64, []),
    "qk_moe_workspace_bytes": (c_uint64, []),
    "qk_moe_workspace_release": (None, []),
    "qk_profile_reset": (None, []),
    "qk_profile_set_enabled": (None, [c_int]),
    "qk_profile_snapshot": (c_int, [c_void_p, c_int]),
}


def _single_hip_runtime() -> None:
    """PyTorch-ROCm bundles its own ``libamdhip64.so.7`` (same soname as /opt/rocm's). Whichever copy is loaded
    first serves the whole process; if ours came first, torch would load a second runtime that sees no device.
    Importing torch (when installed) before the library makes both share torch's runtime."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    _single_hip_runtime()
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m integer_inference_engine_amd.build`")
    so = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(so, name)
        fn.restype = res
        fn.argtypes = args
    return so


@lru_cache(maxsize=1)
def device_available() -> bool:
    """True iff the library loaded and a gfx950 device is usable (rc 0 from ``bonsai_gpu_available``)."""
    return lib().bonsai_gpu_available() == 0


def last_error() -> str:
    v = lib().imie_last_error()
    return v.decode() if v else ""
