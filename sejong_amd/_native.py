"""ctypes binding of libsejong_hip.so (the C ABI in include/sejong_hip.h).

The library is the only compute path: importing this module on a machine
without the built library raises immediately; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsejong_hip.so")

SJ_F32, SJ_F64, SJ_F16, SJ_I32, SJ_BF16 = 0, 1, 2, 3, 4

_P = ctypes.c_void_p
_L = ctypes.c_long
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t
_DB = ctypes.c_double
_U64 = ctypes.c_uint64


class FactoredParam(ctypes.Structure):
    """sj_factored_param of include/sejong_hip.h."""
    _fields_ = [("w", _P), ("dense", _P), ("rows", _L), ("cols", _L), ("decay", _I), ("term_begin", _L),
                ("term_count", _L), ("ld", _L), ("mirror", _P)]


class FactoredTerm(ctypes.Structure):
    """sj_factored_term of include/sejong_hip.h."""
    _fields_ = [("left", _P), ("right", _P), ("tail", _P), ("row_map", _P), ("rank", _L), ("scale", _F),
                ("ld", _L)]


class SejongError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


class ModelConfig(ctypes.Structure):
    _fields_ = [("vocab", _L), ("width", _L), ("layers", _L), ("heads", _L), ("kv_heads", _L),
                ("ffn_width", _L), ("sequence", _L), ("batch", _L), ("norm_epsilon", _F),
                ("rope_theta", _F), ("precision", _I)]


class ExpertConfig(ctypes.Structure):
    _fields_ = [("count", _L), ("top_k", _L), ("ffn_width", _L)]


class HierarchyConfig(ctypes.Structure):
    _fields_ = [("patch_size", _L), ("encoder_width", _L), ("encoder_layers", _L), ("encoder_heads", _L),
                ("encoder_ffn_width", _L), ("decoder_width", _L), ("decoder_layers", _L), ("decoder_heads", _L),
                ("decoder_ffn_width", _L), ("local_window", _L)]


class AdamConfig(ctypes.Structure):
    _fields_ = [("beta1", _F), ("beta2", _F), ("epsilon", _F), ("weight_decay", _F),
                ("clip_norm", _F), ("loss_scale", _F), ("clip_enabled", _I)]


class SgdConfig(ctypes.Structure):
    _fields_ = [("weight_decay", _F), ("clip_norm", _F), ("loss_scale", _F), ("clip_enabled", _I),
                ("vjp_rank", _L), ("vjp_residual_fraction", _DB), ("vjp_block_rows", _L), ("vjp_seed", _U64)]


class AdamStep(ctypes.Structure):
    _fields_ = [("lr", _F), ("beta1", _F), ("beta2", _F), ("eps", _F), ("weight_decay", _F),
                ("inv_b1", _F), ("inv_b2", _F), ("clip_norm", _F), ("loss_scale", _F),
                ("clip_enabled", ctypes.c_int32)]


# name -> (restype, argtypes); int-returning functions are status-checked
SIGNATURES = {
    "sj_status_string": (ctypes.c_char_p, [_I]),
    "sj_last_error": (ctypes.c_char_p, []),
    "sj_device_info": (_I, [ctypes.c_char_p, _S, ctypes.POINTER(_I)]),
    "sj_alloc": (_I, [_S, ctypes.POINTER(_P)]),
    "sj_free": (_I, [_P]),
    "sj_memory_info": (_I, [ctypes.POINTER(_S), ctypes.POINTER(_S)]),
    "sj_upload": (_I, [_P, _P, _S]),
    "sj_download": (_I, [_P, _P, _S]),
    "sj_synchronize": (_I, [_P]),
    "sj_event_create": (_I, [ctypes.POINTER(_P)]),
    "sj_event_destroy": (_I, [_P]),
    "sj_event_record": (_I, [_P, _P]),
    "sj_event_elapsed": (_I, [_P, _P, ctypes.POINTER(_F)]),
    "sj_fill": (_I, [_P, _P, _I, _L, _F]),
    "sj_cast": (_I, [_P, _P, _I, _P, _I, _L]),
    "sj_add": (_I, [_P, _P, _I, _P, _I, _P, _I, _L, _F]),
    "sj_embedding_fwd": (_I, [_P, _P, _I, _P, _P, _I, _L, _L]),
    "sj_embedding_bwd_workspace_bytes": (_S, [_L, _L]),
    "sj_embedding_bwd": (_I, [_P, _P, _P, _P, _L, _L, _L, _P, _S]),
    "sj_rope": (_I, [_P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _F, _I]),
    "sj_rope_table": (_I, [_P, _P, _L, _L, _F]),
    "sj_swiglu_fwd": (_I, [_P, _P, _P, _P, _I, _L]),
    "sj_swiglu_bwd": (_I, [_P, _P, _P, _I, _P, _P, _P, _L]),
    "sj_rmsnorm_fwd": (_I, [_P, _P, _I, _P, _I, _P, _L, _L, _F]),
    "sj_rmsnorm_bwd_workspace_bytes": (_S, [_L, _L]),
    "sj_rmsnorm_bwd": (_I, [_P, _P, _I, _P, _I, _P, _P, _P, _P, _L, _L, _F, _P, _S]),
    "sj_rmsnorm_fwd_t": (_I, [_P, _P, _P, _P, _P, _L, _L, _L, _F]),
    "sj_rmsnorm_bwd_p_workspace_bytes": (_S, [_L, _L]),
    "sj_rmsnorm_bwd_p": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _F, _P, _S]),
    "sj_rmsnorm_bwd_p_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _F]),
    "sj_route_topk": (_I, [_P, _P, _I, _L, _L, _L, _P, _P]),
    "sj_router_topk": (_I, [_P, _P, _L, _P, _L, _L, _L, _L, _P, _P, _P]),
    "sj_route_topk_bwd": (_I, [_P, _P, _I, _P, _P, _P, _P, _L, _L, _L]),
    "sj_route_pack_capacity": (_L, [_L, _L]),
    "sj_route_pack": (_I, [_P, _P, _L, _L, _L, _P, _P, _P, _P, _P, _P, _L]),
    "sj_moe_gather": (_I, [_P, _P, _L, _L, _P, _L, _L, _P, _P, _L]),
    "sj_moe_combine": (_I, [_P, _P, _L, _L, _P, _P, _P, _L, _L, _P, _L, _P, _L]),
    "sj_moe_combine_bwd": (_I, [_P, _P, _L, _L, _P, _P, _L, _L, _P, _L, _P, _P, _P, _P, _L, _P]),
    "sj_moe_gather_bwd": (_I, [_P, _P, _L, _L, _P, _P, _P, _P, _P, _P, _L, _L, _L, _P, _L, _P, _L, _P]),
    "sj_moe_gate_up_fwd": (_I, [_P, _P, _L, _L, _P, _L, _L, _P, _P, _L, _L, _L, _P, _P, _P, _L, _P, _L]),
    "sj_moe_down_fwd": (_I, [_P, _P, _L, _L, _P, _L, _L, _P, _L, _L, _L, _P, _L]),
    "sj_moe_down_bwd_swiglu_p": (_I, [_P, _P, _L, _L, _P, _P, _L, _L, _P, _L, _L, _L, _P, _P, _L, _P, _P, _L, _P,
                                      _P, _L]),
    "sj_moe_gemm_rows": (_I, [_P, _P, _L, _L, _L, _L, _P, _P, _L, _P, _L, _L, _P, _L, _I]),
    "sj_moe_gemm_dw": (_I, [_P, _P, _L, _L, _L, _L, _P, _L, _P, _P, _L, _P, _L, _L]),
    "sj_pvjp_budget": (_I, [_L, _DB, _L, _L, _L, _L, _P, _P, _P]),
    "sj_pvjp_selects_compression": (_I, [_L, _DB, _L, _L, _L, _L, _L, _L]),
    "sj_pvjp_basis_tolerance": (_F, [_L, _L]),
    "sj_pvjp_indices": (_I, [_P, _U64, _L, _L, _L, _L, _L, _L, _P, _P, _P, _P]),
    "sj_pvjp_basis_workspace_bytes": (_S, [_L, _L]),
    "sj_pvjp_basis": (_I, [_P, _P, _I, _L, _L, _P, _L, _F, _P, _P, _S]),
    "sj_pvjp_prepare_workspace_bytes": (_S, [_L, _L, _L]),
    "sj_pvjp_prepare": (_I, [_P, _P, _L, _L, _L, _P, _L, _P, _L, _F, _P, _P, _P, _P, _L, _P, _S]),
    "sj_pvjp_prepare_rows": (_I, [_P, _P, _L, _L, _L, _P, _L, _P, _L, _F, _P, _P, _P, _P, _L, _P, _S]),
    "sj_pvjp_vjp_workspace_bytes": (_S, [_L, _L, _L]),
    "sj_pvjp_vjp": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _L, _L, _P, _L, _P, _S]),
    "sj_pvjp_vjp_rows": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _L, _L, _P, _L, _P, _S]),
    "sj_factored_meta_bytes": (_S, [_P, _L, _L]),
    "sj_factored_pack": (_I, [_P, _L, _P, _L, _P, _S, _P]),
    "sj_factored_apply": (_I, [_P, _P, _L, _I, _F, _F, _P]),
    "sj_sum_f64": (_I, [_P, _P, _L, _P]),
    "sj_attention_fwd_t": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _L, _L, _L, _L, _L, _L]),
    "sj_attention_bwd_p": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _L, _P, _L, _L, _L, _L, _L, _P,
                                _P, _P, _L, _P, _P, _L, _P, _S]),
    "sj_attention_bwd_p_workspace_bytes": (_S, [_L, _L, _L, _L, _L]),
    "sj_gemm_workspace_bytes": (_S, [_L, _L, _L]),
    "sj_gemm": (_I, [_P, _I, _I, _L, _L, _L, _P, _I, _L, _P, _I, _L, _P, _I, _L, _I, _P, _S]),
    "sj_qkv_fwd": (_I, [_P, _P, _L, _L, _L, _P, _L, _P, _L, _P, _L, _L, _L, _P, _L, _P, _L, _P, _L, _I,
                        _P, _L, _L]),
    "sj_gate_up_fwd": (_I, [_P, _P, _L, _L, _L, _P, _L, _P, _L, _L, _P, _P, _P, _L, _I]),
    "sj_linear_residual_fwd": (_I, [_P, _P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _L, _I]),
    "sj_down_bwd_swiglu": (_I, [_P, _P, _L, _L, _L, _P, _L, _L, _P, _P, _L, _I, _P, _L]),
    "sj_gemm_planes_workspace_bytes": (_S, [_L, _L, _L]),
    "sj_gemm_planes": (_I, [_P, _L, _L, _L, _P, _P, _L, _P, _P, _L, _P, _I, _L, _I, _P, _S]),
    "sj_attention_fwd_tt": (_I, [_P, _P, _L, _L, _L, _L, _L, _L, _L, _L, _P, _L, _P, _P, _P, _L]),
    "sj_attention_bwd_tt_workspace_bytes": (_S, [_L, _L, _L, _L, _L]),
    "sj_attention_bwd_tt_counter_bytes": (_S, [_L, _L]),
    "sj_attention_bwd_tt": (_I, [_P, _P, _L, _L, _P, _L, _P, _P, _P, _L, _P, _L, _L, _L, _L, _L, _L, _P,
                                 _P, _P, _L, _P, _P, _L, _P, _S]),
    "sj_attention_bwd_plan": (_I, [_L, _L, _L, _I, _P, _L, _P]),
    "sj_gemm_planes_tn": (_I, [_P, _L, _L, _L, _P, _P, _L, _P, _P, _L, _P, _I, _L, _I, _P, _S]),
    "sj_moe_gemm_dw_tn": (_I, [_P, _P, _L, _L, _L, _L, _P, _L, _P, _P, _L, _P, _L, _L]),
    "sj_gemm_planes_split_out": (_I, [_P, _L, _L, _L, _P, _P, _L, _P, _L, _P, _P, _L, _P, _P, _L, _P, _L, _P, _L]),
    "sj_qkv_fwd_t": (_I, [_P, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _P, _L, _L, _P, _L]),
    "sj_gate_up_fwd_t": (_I, [_P, _P, _L, _L, _L, _P, _P, _L, _L, _P, _P, _P, _L, _P, _L]),
    "sj_linear_residual_fwd_t": (_I, [_P, _P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _L]),
    "sj_down_bwd_swiglu_p": (_I, [_P, _P, _P, _L, _L, _L, _P, _L, _L, _P, _P, _L, _P, _P, _L, _P, _P, _L]),
    "sj_attention_fwd": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _L, _P, _I, _L, _L, _L, _L, _L, _L]),
    "sj_attention_bwd": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _L, _P, _L, _P, _L, _P, _L, _P,
                              _I, _L, _L, _L, _L, _L, _L, _P]),
    "sj_cross_entropy": (_I, [_P, _P, _L, _P, _P, _P, _L, _L, _L, _P, _F]),
    "sj_loss_summary": (_I, [_P, _P, _L, _P, _L, _F]),
    "sj_sum_squares_workspace_bytes": (_S, [_L]),
    "sj_sum_squares": (_I, [_P, _P, _L, _P, _P, _S]),
    "sj_adamw": (_I, [_P, _P, _P, _P, _P, _L, _F, _F, _F, _F, _F, _F, _F, _F]),
    "sj_adamw_multi": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _P, _P, _P]),
    "sj_gather_rows": (_I, [_P, _P, _I, _L, _P, _L, _L, _P, _I]),
    "sj_gather_rows_bwd": (_I, [_P, _P, _P, _L, _L, _P, _L, _L]),
    "sj_bias_add": (_I, [_P, _P, _L, _P, _P, _L, _L, _L]),
    "sj_bias_reduce": (_I, [_P, _P, _L, _L, _L, _P]),
    "sj_patch_pool": (_I, [_P, _P, _I, _L, _L, _L, _L, _P]),
    "sj_patch_pool_bwd": (_I, [_P, _P, _L, _L, _L, _L, _P]),
    "sj_patch_broadcast": (_I, [_P, _P, _P, _I, _L, _L, _L, _L, _P]),
    "sj_patch_broadcast_bwd": (_I, [_P, _P, _L, _L, _L, _L, _P, _P]),
    "sj_model_create": (_I, [ctypes.POINTER(ModelConfig), ctypes.POINTER(AdamConfig), _P, ctypes.POINTER(_P)]),
    "sj_safetensors_write": (_I, [ctypes.c_char_p, _L, _P, _P, _P, _P]),
    "sj_safetensors_header": (_I, [ctypes.c_char_p, _P, _S, ctypes.POINTER(_S)]),
    "sj_safetensors_read": (_I, [ctypes.c_char_p, ctypes.c_char_p, _P, _L]),
    "sj_checkpoint_save": (_I, [ctypes.c_char_p, ctypes.c_char_p, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P]),
    "sj_blake3_state_bytes": (_S, []),
    "sj_blake3_init": (_I, [_P]),
    "sj_blake3_update": (_I, [_P, _P, _S]),
    "sj_blake3_finalize": (_I, [_P, _P]),
    "sj_model_create_experts": (_I, [ctypes.POINTER(ModelConfig), ctypes.POINTER(ExpertConfig),
                                     ctypes.POINTER(AdamConfig), _P, ctypes.POINTER(_P)]),
    "sj_model_create_hierarchy": (_I, [ctypes.POINTER(ModelConfig), ctypes.POINTER(HierarchyConfig),
                                       ctypes.POINTER(AdamConfig), _P, ctypes.POINTER(_P)]),
    "sj_model_create_sgd": (_I, [ctypes.POINTER(ModelConfig), ctypes.POINTER(SgdConfig), _P, ctypes.POINTER(_P)]),
    "sj_model_materialize_grads": (_I, [_P]),
    "sj_model_create_value": (_I, [ctypes.POINTER(ModelConfig), _L, ctypes.POINTER(AdamConfig),
                                   ctypes.POINTER(SgdConfig), _P, ctypes.POINTER(_P)]),
    "sj_model_set_value_batch": (_I, [_P, _P, _P, _P]),
    "sj_model_vjp_info": (_I, [_P, ctypes.POINTER(_L), ctypes.POINTER(_L), ctypes.POINTER(_L), ctypes.POINTER(_L),
                               ctypes.POINTER(_U64)]),
    "sj_model_set_vjp_rng": (_I, [_P, _U64]),
    "sj_model_steps": (_L, [_P]),
    "sj_model_destroy": (_I, [_P]),
    "sj_model_param_tensors": (_L, [_P]),
    "sj_model_param_count": (_L, [_P]),
    "sj_model_param_info": (_I, [_P, _L, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_L),
                                 ctypes.POINTER(_L), ctypes.POINTER(_L)]),
    "sj_model_set_params": (_I, [_P, _P]),
    "sj_model_get_params": (_I, [_P, _P]),
    "sj_model_get_grads": (_I, [_P, _P]),
    "sj_model_get_adam_state": (_I, [_P, _P, _P, ctypes.POINTER(_L)]),
    "sj_model_set_adam_state": (_I, [_P, _P, _P, _L]),
    "sj_model_set_batch": (_I, [_P, _P, _P, _I]),
    "sj_model_set_batches": (_I, [_P, _P, _P, _L]),
    "sj_model_forward_backward": (_I, [_P]),
    "sj_model_train_step": (_I, [_P, _F]),
    "sj_model_use_graph": (_I, [_P, _I]),
    "sj_model_forward": (_I, [_P]),
    "sj_cache_create": (_I, [_P, _L, ctypes.POINTER(_P)]),
    "sj_cache_destroy": (_I, [_P]),
    "sj_cache_reset": (_I, [_P]),
    "sj_cache_length": (_L, [_P]),
    "sj_model_forward_cached": (_I, [_P, _P, _P, _L, _P]),
    "sj_attention_fwd_cached": (_I, [_P, _P, _L, _P, _P, _L, _L, _I, _L, _L, _L, _L, _L, _L, _P, _L]),
    "sj_model_read_loss": (_I, [_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "sj_model_profile": (_I, [_P, _I]),
    "sj_model_profile_collect": (_L, [_P]),
    "sj_model_profile_kernel": (_I, [_P, _L, ctypes.POINTER(ctypes.c_char_p)]),
    "sj_model_profile_entry": (_I, [_P, _L, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(_L)]),
    "sj_model_activation_count": (_L, [_P]),
    "sj_model_export_activations": (_I, [_P, _P]),
    "sj_model_buffer": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(_L)]),
}

# functions whose int result is a status (sj_attention_bwd_plan returns a count)
STATUS_FUNCS = {n for n, (r, _) in SIGNATURES.items()
                if r is _I and n not in ("sj_status_string", "sj_attention_bwd_plan")}

_lib = None


def load(path: str | None = None):
    """Load the library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -m sejong_amd.build` "
                          "(there is no CPU fallback for the HIP path)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().sj_last_error().decode()


def check(status: int):
    if status != 0:
        raise SejongError(status, last_error())


class _Checked:
    """lib.<name>(...) raising SejongError on a non-zero status."""

    def __getattr__(self, name):
        fn = getattr(load(), name)
        if name not in STATUS_FUNCS:
            return fn

        def call(*args):
            check(fn(*args))
        return call


api = _Checked()
