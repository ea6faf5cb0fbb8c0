"""ctypes binding of libane_hip.so (the C-ABI declared in include/ane_hip.h).

The library is built in-tree (``autoresearch-go-ane_amd/csrc/Makefile``) and
loaded from this directory.  There is no fallback: if the library is missing
or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libane_hip.so")

ANE_OK = 0
ANE_ERR_CLOSED = -1
ANE_ERR_ARG = -2
ANE_ERR_HIP = -3
ANE_ERR_NOMEM = -4
ANE_ERR_STATE = -5

ARCH = {"nanochat": 0, "llama2": 1}
GRAD = {"compat": 0, "true": 1}
PROF_CLASSES = ["qkv_gemm", "wo_gemm", "ffn_up_gemm", "ffn_down_gemm", "classifier_gemm", "attention",
                "rmsnorm", "other"]


class ModelCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32), ("layers", C.c_int32),
                ("vocab", C.c_int32), ("seq", C.c_int32), ("arch", C.c_int32), ("grad_mode", C.c_int32),
                ("rope_theta", C.c_double)]


class Options(C.Structure):
    _fields_ = [("accum_steps", C.c_int32), ("lr", C.c_float), ("seed", C.c_int64),
                ("adam_beta1", C.c_float), ("adam_beta2", C.c_float), ("adam_eps", C.c_float),
                ("weight_decay", C.c_float), ("grad_clip", C.c_float), ("loss_scale", C.c_float),
                ("embed_lr_mult", C.c_float), ("scalar_lr_mult", C.c_float), ("lambda_lr_mult", C.c_float),
                ("lambda_beta1", C.c_float), ("lambda_beta2", C.c_float), ("max_batch", C.c_int32),
                ("device", C.c_int32)]


class State(C.Structure):
    _fields_ = [("token_pos", C.c_uint64), ("last_loss", C.c_float), ("cum_train_ms", C.c_double),
                ("cum_wall_ms", C.c_double), ("cum_steps", C.c_uint32), ("cum_batches", C.c_uint32),
                ("adam_t", C.c_uint32), ("pending_steps", C.c_uint32)]


class StepResult(C.Structure):
    _fields_ = [("loss", C.c_float)] + [(n, C.c_int64) for n in (
        "step_ns", "compile_ns", "startup_compile_ns", "ane_eval_ns", "cpu_work_ns", "weight_refresh_ns",
        "final_head_ns", "embed_grad_ns", "rms_dw_ns", "dw_gemm_ns", "dw_wait_ns", "adam_ns")]


class DecodeCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32), ("kv_heads", C.c_int32),
                ("layers", C.c_int32), ("vocab", C.c_int32), ("max_batch", C.c_int32), ("max_ctx", C.c_int32),
                ("rope_theta", C.c_double), ("device", C.c_int32)]


class MoeCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden", C.c_int32), ("experts", C.c_int32), ("top_k", C.c_int32),
                ("max_tokens", C.c_int32), ("device", C.c_int32)]


class LayerWeights(C.Structure):
    """ane_layer_weights (include/ane_objects.h)."""
    _fields_ = [(n, C.POINTER(C.c_float)) for n in ("wq", "wk", "wv", "wo", "w1", "w2")]


LAYER_TAPS = ("x_norm", "q", "k", "v", "att_out", "x2", "x2_norm", "h1", "gate")


class LayerCache(C.Structure):
    """ane_layer_cache (include/ane_objects.h)."""
    _fields_ = [(n, C.POINTER(C.c_float)) for n in LAYER_TAPS] + [("att_taps_ready", C.c_int32),
                                                                  ("ffn_taps_ready", C.c_int32)]


class ProfEntry(C.Structure):
    _fields_ = [("launches", C.c_int64), ("ms", C.c_double), ("flops", C.c_double), ("bytes", C.c_double)]


# every exported symbol of include/ane_hip.h with (restype, argtypes)
_fp = C.POINTER(C.c_float)
_u16 = C.POINTER(C.c_uint16)
_u64 = C.POINTER(C.c_uint64)
_eng = C.c_void_p
SIGNATURES = {
    "ane_open": (C.c_int, [C.POINTER(ModelCfg), C.POINTER(Options), C.POINTER(C.c_void_p)]),
    "ane_close": (None, [_eng]),
    "ane_destroy": (None, [_eng]),
    "ane_last_error": (C.c_char_p, [_eng]),
    "ane_param_count": (C.c_int64, [C.POINTER(ModelCfg)]),
    "ane_param_layout": (C.c_int, [C.POINTER(ModelCfg), C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_int]),
    "ane_set_params": (C.c_int, [_eng, _fp, C.c_int64]),
    "ane_get_params": (C.c_int, [_eng, _fp, C.c_int64]),
    "ane_set_tokens": (C.c_int, [_eng, _u16, C.c_int64]),
    "ane_eval_logits": (C.c_int, [_eng, _u16, C.c_int64, _fp]),
    "ane_eval_loss": (C.c_int, [_eng, _u16, _u16, C.c_int32, _fp, _fp]),
    "ane_eval_loss_windows": (C.c_int, [_eng, _u64, C.c_int32, _fp, _fp]),
    "ane_step": (C.c_int, [_eng, C.POINTER(StepResult)]),
    "ane_train_batch": (C.c_int, [_eng, C.c_int32, C.POINTER(StepResult)]),
    "ane_flush": (C.c_int, [_eng, C.POINTER(C.c_int64)]),
    "ane_lr": (C.c_float, [_eng]),
    "ane_set_lr": (C.c_int, [_eng, C.c_float]),
    "ane_get_state": (C.c_int, [_eng, C.POINTER(State)]),
    "ane_load_state": (C.c_int, [_eng, C.POINTER(State)]),
    "ane_grads": (C.c_int, [_eng, _u16, _u16, C.c_int32, _fp, _fp]),
    "ane_set_grads": (C.c_int, [_eng, _fp, C.c_int64, C.c_uint32]),
    "ane_get_opt_state": (C.c_int, [_eng, _fp, _fp, C.c_int64]),
    "ane_set_opt_state": (C.c_int, [_eng, _fp, _fp, C.c_int64]),
    "ane_get_accum_grads": (C.c_int, [_eng, _fp, C.c_int64]),
    "ane_seed_sampler": (C.c_int, [_eng, C.c_int64]),
    "ane_profile_enable": (C.c_int, [_eng, C.c_int]),
    "ane_profile_read": (C.c_int, [_eng, C.POINTER(ProfEntry), C.c_int, C.c_int]),
    "ane_sync": (C.c_int, [_eng]),
    "ane_debug_gemm": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _u16, _u16, C.c_void_p,
                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "ane_debug_gemm_epi": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _u16, _u16, C.c_void_p, C.c_void_p,
                                     _fp, _fp, C.c_float, C.c_float, C.c_int, C.c_int, C.c_int, C.c_int]),
    "ane_debug_gemm_norm": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _u16, _u16, _fp, _u16, _fp, _fp, _fp,
                                      C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "ane_debug_attention": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, C.c_float, C.c_int, _u16,
                                      _u16, _fp]),
    "ane_debug_transpose2": (C.c_int, [C.c_int, C.c_int, _u16, _u16, C.c_int, C.c_int, _u16, _u16]),
    "ane_debug_norm_bwd": (C.c_int, [C.c_int, C.c_int, _fp, _fp, _fp, _fp, C.c_float, _fp, _u16, _fp, C.c_int]),
    "ane_debug_classifier": (C.c_int, [C.c_int, C.c_int, C.c_int, _u16, _u16, _u16, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, _fp, _fp, _fp, _fp, _fp, _u16, _u16]),
    "ane_debug_last_error": (C.c_char_p, []),
    "ane_kernel_abi": (C.c_int, [C.c_char_p, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_int]),
    "ane_debug_gemm_bench": (C.c_int, [C.c_int] * 12 + [_u16, _u16, _fp]),
    "ane_head_loss": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]),
    "ane_head_loss_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]),
    "ane_op_last_error": (C.c_char_p, []),
    "ane_decode_open": (C.c_int, [C.POINTER(DecodeCfg), C.POINTER(C.c_void_p)]),
    "ane_decode_destroy": (None, [_eng]),
    "ane_decode_last_error": (C.c_char_p, [_eng]),
    "ane_decode_param_count": (C.c_int64, [C.POINTER(DecodeCfg)]),
    "ane_decode_set_params": (C.c_int, [_eng, _fp, C.c_int64]),
    "ane_decode_prefill": (C.c_int, [_eng, _u16, C.c_int32, C.c_int32, _u16, _fp]),
    "ane_decode_step": (C.c_int, [_eng, _u16, _u16, _fp]),
    "ane_decode_generate": (C.c_int, [_eng, C.c_int32, _u16]),
    "ane_decode_position": (C.c_int32, [_eng]),
    "ane_decode_last_ms": (C.c_double, [_eng]),
    "ane_decode_fused_chain": (C.c_int32, [_eng]),
    "ane_decode_debug_fill_cache": (C.c_int, [_eng, C.c_int]),
    "ane_moe_open": (C.c_int, [C.POINTER(MoeCfg), C.POINTER(C.c_void_p)]),
    "ane_moe_destroy": (None, [_eng]),
    "ane_moe_last_error": (C.c_char_p, [_eng]),
    "ane_moe_param_count": (C.c_int64, [C.POINTER(MoeCfg)]),
    "ane_moe_set_params": (C.c_int, [_eng, _fp, C.c_int64]),
    "ane_moe_load_input": (C.c_int, [_eng, _fp, C.c_int32]),
    "ane_moe_run": (C.c_int, [_eng]),
    "ane_moe_read_output": (C.c_int, [_eng, _fp, C.POINTER(C.c_int32), _fp]),
    "ane_moe_last_ms": (C.c_double, [_eng]),
    # the per-object seam (include/ane_objects.h)
    "ane_seam_last_error": (C.c_char_p, []),
    "ane_layer_forward_open": (C.c_int, [C.c_int32] * 4 + [C.POINTER(LayerWeights), C.POINTER(C.c_void_p)]),
    "ane_layer_forward_run": (C.c_int, [_eng, _fp, _fp]),
    "ane_layer_forward_run_taps": (C.c_int, [_eng, _fp, _fp, C.POINTER(LayerCache)]),
    "ane_layer_forward_refresh": (C.c_int, [_eng, C.POINTER(LayerWeights)]),
    "ane_layer_forward_close": (None, [_eng]),
    "ane_layer_forward_destroy": (None, [_eng]),
    "ane_layer_backward_open": (C.c_int, [C.c_int32] * 4 + [C.POINTER(LayerWeights), C.POINTER(C.c_void_p)]),
    "ane_layer_backward_run_attention": (C.c_int, [_eng] + [_fp] * 8),
    "ane_layer_backward_run_ffn": (C.c_int, [_eng] + [_fp] * 4),
    "ane_layer_backward_refresh": (C.c_int, [_eng, C.POINTER(LayerWeights)]),
    "ane_layer_backward_close": (None, [_eng]),
    "ane_layer_backward_destroy": (None, [_eng]),
    "ane_offload_open": (C.c_int, [C.c_int32] * 3 + [_fp, C.c_int32, C.POINTER(C.c_void_p)]),
    "ane_offload_has": (C.c_int, [_eng, C.c_int32]),
    "ane_offload_disable": (None, [_eng, C.c_int32]),
    "ane_offload_run_rms_forward": (C.c_int, [_eng, _fp, _fp]),
    "ane_offload_run_classifier_forward": (C.c_int, [_eng, _fp, _fp]),
    "ane_offload_run_classifier_softmax": (C.c_int, [_eng, _fp, _fp]),
    "ane_offload_run_softmax": (C.c_int, [_eng, _fp]),
    "ane_offload_run_classifier_backward": (C.c_int, [_eng, _fp, _fp]),
    "ane_offload_run_rms_backward": (C.c_int, [_eng, _fp, _fp, _fp]),
    "ane_offload_refresh": (C.c_int, [_eng, _fp]),
    "ane_offload_close": (None, [_eng]),
    "ane_offload_destroy": (None, [_eng]),
}

_lib = None


def load():
    """Loads libane_hip.so once; raises if it is missing or incomplete."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libane_hip.so not built ({LIB_PATH}); run __graft_entry__.build() or "
                           "make -C autoresearch-go-ane_amd/csrc")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def model_cfg(cfg) -> ModelCfg:
    return ModelCfg(cfg.dim, cfg.hidden, cfg.heads, cfg.layers, cfg.vocab, cfg.seq, ARCH[cfg.arch],
                    GRAD[cfg.grad_mode], float(cfg.rope_theta))
