"""tinytorch on MI355X (gfx950): loader for the in-tree C-ABI library.

`lib()` returns the ctypes handle of build/libtinytorch.so with every
signature of include/tensor.h, include/autograd.h and include/tt_hip.h
declared.  The library is built by `make lib` (or `__graft_entry__.build()`);
nothing here compiles.  There is no CPU fallback: on a machine without a
usable GPU, `require_gpu()` raises and every op returns NULL.
"""
import ctypes
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "build")
LIB_PATH = os.path.join(BUILD, "libtinytorch.so")

F32P = ctypes.POINTER(ctypes.c_float)
I64P = ctypes.POINTER(ctypes.c_long)
VP = ctypes.c_void_p

_LIB = None

# (name, restype, argtypes) for every exported symbol the headers declare
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_SZ = ctypes.c_size_t
SIGNATURES = [
    # tensor.h
    ("tt_new", VP, [I64P, _I]),
    ("tt_fromdata", VP, [F32P, I64P, _I]),
    ("tt_retain", VP, [VP]),
    ("tt_release", None, [VP]),
    ("tt_data", F32P, [VP]),
    ("tt_numel", _L, [VP]),
    ("tt_ndim", _I, [VP]),
    ("tt_shape", None, [VP, I64P]),
    ("tt_strides", None, [VP, I64P]),
    ("tt_add", VP, [VP, VP]),
    ("tt_mul", VP, [VP, VP]),
    ("tt_addscalar", VP, [VP, _F]),
    ("tt_mulscalar", VP, [VP, _F]),
    ("tt_matmul", VP, [VP, VP]),
    ("tt_matmul_fast", VP, [VP, VP]),
    ("tt_matmul_omp", VP, [VP, VP, _I]),
    ("tt_relu", VP, [VP]),
    ("tt_softmax", VP, [VP]),
    ("tt_reshape", VP, [VP, I64P, _I]),
    ("tt_conv2d", VP, [VP, VP, VP, _I, _I, _I, _I]),
    ("tt_maxpool2d", VP, [VP, _I, _I, _I, _I]),
    ("tt_avgpool2d", VP, [VP, _I, _I, _I, _I]),
    ("tt_sgemm_rowmajor", _I, [_I, _I, _I, F32P, F32P, F32P, _I]),
    # autograd.h
    ("ag_leaf", VP, [VP, _I]),
    ("ag_add", VP, [VP, VP]),
    ("ag_mul", VP, [VP, VP]),
    ("ag_addscalar", VP, [VP, _F]),
    ("ag_mulscalar", VP, [VP, _F]),
    ("ag_matmul", VP, [VP, VP]),
    ("ag_relu", VP, [VP]),
    ("ag_softmax", VP, [VP]),
    ("ag_padones", VP, [VP]),
    ("ag_reshape", VP, [VP, I64P, _I]),
    ("ag_conv2d", VP, [VP, VP, VP, _I, _I, _I, _I]),
    ("ag_maxpool2d", VP, [VP, _I, _I, _I, _I]),
    ("ag_avgpool2d", VP, [VP, _I, _I, _I, _I]),
    ("ag_value", VP, [VP]),
    ("ag_grad", VP, [VP]),
    ("ag_requires_grad", _I, [VP]),
    ("ag_backward", None, [VP]),
    ("ag_backward_from", None, [VP, F32P, _SZ]),
    ("ag_release", None, [VP]),
    ("ag_retain", VP, [VP]),
    ("ag_softmax_ce", VP, [VP, ctypes.POINTER(ctypes.c_int), _L]),
    ("ag_softmax_ce_probs", VP, [VP]),
    ("ag_backward_from_tensor", None, [VP, VP]),
    ("ag_sgd_step", _I, [VP, _F]),
    ("ag_sgd_step_many", _I, [ctypes.POINTER(VP), _I, _F]),
    ("ag_optim_sgd_momentum", VP, [ctypes.c_double, ctypes.c_double]),
    ("ag_optim_adam", VP, [ctypes.c_double] * 4),
    ("ag_optim_step", _I, [VP, ctypes.POINTER(VP), _I]),
    ("ag_optim_steps", _L, [VP]),
    ("ag_optim_release", None, [VP]),
    ("ag_optim_set_lr", _I, [VP, ctypes.c_double]),
    ("ag_optim_lr", ctypes.c_double, [VP]),
    # tt_data.h: device-resident datasets
    ("tt_idx_probe", _I, [ctypes.c_char_p, ctypes.POINTER(_I), ctypes.POINTER(_L)]),
    ("tt_dataset_idx", VP, [ctypes.c_char_p, ctypes.c_char_p]),
    ("tt_dataset_cifar10_bin", VP, [ctypes.POINTER(ctypes.c_char_p), _I]),
    ("tt_dataset_from_u8", VP, [VP, VP, _L, _I, _I, _I]),
    ("tt_dataset_len", _L, [VP]),
    ("tt_dataset_shape", _I, [VP, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    ("tt_dataset_labels", _I, [VP, VP]),
    ("tt_dataset_batch", VP, [VP, VP, _L, F32P, F32P, _I, VP]),
    ("tt_dataset_release", None, [VP]),
    # tt_hip.h: runtime
    ("tth_available", _I, []),
    ("tth_device_name", _I, [ctypes.c_char_p, _I]),
    ("tth_stream", VP, []),
    ("tth_sync", _I, []),
    ("tth_last_error", _I, []),
    ("tth_malloc", VP, [_SZ]),
    ("tth_free", None, [VP]),
    ("tth_release_cache", None, []),
    ("tth_bytes_in_use", _SZ, []),
    ("tth_fail_alloc_after", _I, [ctypes.c_long]),
    ("tth_h2d", _I, [VP, VP, _SZ]),
    ("tth_d2h", _I, [VP, VP, _SZ]),
    ("tt_dev", VP, [VP]),
    ("tth_event_create", VP, []),
    ("tth_event_record", _I, [VP]),
    ("tth_event_elapsed_ms", _F, [VP, VP]),
    ("tth_event_destroy", None, [VP]),
    # tt_hip.h: kernels (device pointers)
    ("tth_gemm_config", _I, [_I, _I]),
    ("tt_k_gemm", _I, [_I, _I, _I, VP, _I, _I, VP, _I, _I, VP, _I]),
    ("tt_k_head_bwd", _I, [VP, _I, _I, VP, _I, VP, VP, VP, VP, VP, VP]),
    ("tt_k_head_bwd_pool", _I, [VP, _I, _I, VP, _I, VP, VP, VP, VP, VP, VP, VP, _I, _I, _I]),
    ("tt_k_gemm_tn_padones", _I, [_I, _I, _I, VP, VP, VP]),
    ("tt_k_gemm_bias_ce", _I, [_I, _I, _I, VP, VP, VP, VP, VP, VP, VP, VP, ctypes.c_float]),
    ("tt_k_ce_mean_rows", _I, [VP, VP, _I]),
    ("tt_k_matmul_bwd_small", _I, [VP, _I, _I, VP, _I, VP, VP, VP, VP, VP, VP]),
    ("tt_k_matmul_naive", _I, [VP, VP, VP, _I, _I, _I]),
    ("tt_k_gemm_noalloc", _I, [_I, _I, _I, VP, _I, _I, VP, _I, _I, VP, _I]),
    ("tt_k_conv_fwd", _I, [_I, _I, _L, _I, VP, VP, VP, VP]),
    ("tt_k_conv_dw", _I, [_I, _I, _L, _I, VP, VP, VP]),
    ("tt_k_conv_dcol", _I, [_I, _I, _L, _I, VP, VP, VP]),
    ("tt_k_conv_dw_bias", _I, [_I, _I, _L, _I, VP, VP, VP, VP]),
    ("tt_k_fill", _I, [VP, _L, _F]),
    ("tt_k_copy", _I, [VP, VP, _L]),
    ("tt_k_add_inplace", _I, [VP, VP, _L]),
    ("tt_k_relu_fwd", _I, [VP, VP, _L]),
    ("tt_k_relu_bwd", _I, [VP, VP, VP, _L]),
    ("tt_k_binary", _I, [VP, VP, VP, _L, _I]),
    ("tt_k_scalar", _I, [VP, VP, _L, _F, _I]),
    ("tt_k_softmax_fwd", _I, [VP, VP, _L, _I]),
    ("tt_k_softmax_bwd", _I, [VP, VP, VP, _L, _I]),
    ("tt_k_softmax_ce", _I, [VP, VP, VP, VP, VP, _L, _I, _F]),
    ("tt_k_softmax_ce_mean", _I, [VP, VP, VP, VP, VP, _L, _I, _F]),
    ("tt_k_softmax_ce_mean_hostlab", _I, [VP, VP, VP, VP, VP, _L, _I, _F]),
    ("tt_k_scale_by_dev", _I, [VP, VP, VP, _L]),
    ("tt_k_padones_fwd", _I, [VP, VP, _L, _L]),
    ("tt_k_copy_padones_fwd", _I, [VP, VP, VP, _L, _L]),
    ("tt_k_relu_padones_fwd", _I, [VP, VP, VP, _L, _L]),
    ("tt_k_gemm_relu_pad", _I, [_I, _I, _I, VP, VP, VP, VP, VP]),
    ("tt_k_gemm_bias_relu_pad", _I, [_I, _I, _I, VP, VP, VP, VP, VP, VP]),
    ("tt_k_padones_bwd2", _I, [VP, VP, VP, _L, _L]),
    ("tt_k_padones_bwd", _I, [VP, VP, _L, _L]),
    ("tt_k_padones_relu_bwd", _I, [VP, VP, VP, VP, _L, _L]),
    ("tt_k_im2col", _I, [VP, VP] + [_I] * 12),
    ("tt_k_im2col_ones", _I, [VP, VP] + [_I] * 12),
    ("tt_k_col2im", _I, [VP, VP] + [_I] * 12),
    ("tt_k_bias_grad", _I, [VP, VP, _I, _I, _I]),
    ("tt_k_maxpool_fwd", _I, [VP, VP] + [_I] * 10),
    ("tt_k_maxpool_bwd", _I, [VP, VP, VP] + [_I] * 10),
    ("tt_k_maxpool2x2_relu_bwd", _I, [VP, VP, VP, VP] + [_I] * 6),
    ("tt_k_maxpool2x2_prerelu_bwd", _I, [VP, VP, VP, VP] + [_I] * 6),
    ("tt_k_maxpool2x2_code_relu_bwd", _I, [VP, VP, VP] + [_I] * 6),
    ("tt_k_avgpool_fwd", _I, [VP, VP] + [_I] * 10),
    ("tt_k_avgpool_bwd", _I, [VP, VP] + [_I] * 10),
    ("tt_k_sgd", _I, [VP, VP, _L, _F]),
    ("tt_k_sgd_multi", _I, [ctypes.POINTER(VP), ctypes.POINTER(VP), ctypes.POINTER(_L), _I, _F]),
    ("tth_conv_config", _I, [_L]),
    ("tth_gemm_direct", _I, [_I]),
    ("tth_gemm_mid", _I, [_I]),
    ("tth_gemm_mid_force", _I, [_I]),
    ("tth_gemm_small", _I, [_I]),
    ("tth_gemm_t16", _I, [_I]),
    ("tth_ce_spec_count", _L, []),
    ("tt_k_conv2d_fwd_implicit", _I, [VP, VP, VP, VP] + [_I] * 13),
    ("tt_k_conv2d_dw_implicit", _I, [VP, VP, VP, VP] + [_I] * 13),
    ("tt_k_conv2d_dx_implicit", _I, [VP, VP, VP] + [_I] * 13),
    ("tth_conv_lds", _I, [_I]),
    ("tth_conv_relu_fuse", _I, [_I]),
    ("tth_conv_chain", _I, [_I]),
    ("tth_conv_dwt", _I, [_I]),
    ("tt_k_conv2d_lds_plan", _I, [_I] * 13),
    ("tt_k_conv2d_fwd_lds", _I, [VP, VP, VP, VP] + [_I] * 13),
    ("tt_k_conv2d_relu_fwd_lds", _I, [VP, VP, VP, VP, VP] + [_I] * 13),
    ("tt_k_conv2d_relu_pool_fwd_lds", _I, [VP] * 9 + [_I] * 13),
    ("tt_k_conv2d_dw_lds", _I, [VP, VP, VP, VP] + [_I] * 13),
    ("tt_k_conv2d_chain_fwd", _I, [VP] * 14 + [_I] + [VP] + [_I] * 6),
    ("tt_k_conv2d_chain_bwd", _I, [VP] * 10 + [_I] * 2),
    ("tt_k_conv2d_dw_lds_pooled", _I, [VP] * 5 + [_I] * 13),
    ("tt_k_conv2d_dx_lds", _I, [VP, VP, VP] + [_I] * 13),
    ("tt_k_gather_u8_norm", _I, [VP, _L, _L, _L, _I, VP, _L, F32P, F32P, VP]),
    ("tt_k_momentum_multi", _I, [ctypes.POINTER(VP)] * 3 + [ctypes.POINTER(_L), _I, _F, _F]),
    ("tt_k_adam_multi", _I, [ctypes.POINTER(VP)] * 4 + [ctypes.POINTER(_L), _I] + [_F] * 5
     + [ctypes.c_double]),
]


def lib():
    """ctypes handle of build/libtinytorch.so with all signatures declared."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `make lib` or __graft_entry__.build()")
        h = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _LIB = h
    return _LIB


def gpu_available():
    return bool(lib().tth_available())


def require_gpu():
    """Raise unless the HIP backend has a usable GPU (no CPU fallback exists)."""
    if not gpu_available():
        raise RuntimeError("tinytorch_amd: no usable GPU; the HIP backend has no CPU fallback")


def device_name():
    buf = ctypes.create_string_buffer(64)
    if lib().tth_device_name(buf, 64) != 0:
        return None
    return buf.value.decode()
