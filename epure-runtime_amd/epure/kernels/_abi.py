"""ctypes binding of ``libepure_hip.so`` (the C ABI in ``include/epure_hip.h``).

Loaded after torch so the library resolves to the HIP runtime torch already
mapped (both carry the soname ``libamdhip64.so.7``): streams and device
pointers from torch are then valid handles for the library.
"""
import ctypes
import os

import torch

LIB_NAME = "libepure_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib",
                        LIB_NAME)

ABI_VERSION = 1
F32, F16, BF16 = 0, 1, 2
FLAG_ACCUMULATE = 1
OK = 0

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_i64, _c_int, _p, _sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t

_SIGS = {
    "ep_abi_version": (_c_int, []),
    "ep_hip_available": (_c_int, []),
    "ep_last_error": (ctypes.c_char_p, []),
    "ep_dequant_matmul_workspace": (_sz, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "ep_dequant_matmul": (_c_int, [
        _p, _c_int, _c_i64,                      # x, x_dtype, ldx
        _p, _p, _c_int, _c_i64,                  # packed, scale, scale_dtype, ld_scale
        _p, _c_int, _c_int, _c_int,              # cb, cb_dtype, levels, group
        _c_i64, _c_i64, _c_i64,                  # M, N, K
        _p, _c_int, _c_i64, _c_int,              # y, y_dtype, ldy, flags
        _p, _sz, _p]),                           # workspace, bytes, stream
    "ep_read_probe": (_c_int, [_p, _c_i64, _p, _c_int, _p]),
    "ep_noalloc_scratch_bytes": (_sz, []),
    "ep_dequant_matmul_noalloc": (_c_int, [
        _p, _c_int, _c_i64,                      # x, x_dtype, ldx
        _p, _p, _c_int, _c_i64,                  # packed, scale, scale_dtype, ld_scale
        _p, _c_int, _c_int, _c_int,              # cb, cb_dtype, levels, group
        _c_i64, _c_i64, _c_i64,                  # M, N, K
        _p, _c_int, _c_i64, _c_int,              # y, y_dtype, ldy, flags
        _p]),                                    # stream
    "ep_expert_matmul": (_c_int, [
        _p, _c_int, _c_i64, _p, _c_i64,         # x, x_dtype, ldx, expert_ids (int32), T
        _p, _p, _c_int, _c_i64,                  # packed, scale, scale_dtype, ld_scale
        _p, _c_int, _c_int, _c_int,              # cb, cb_dtype, levels, group
        _c_i64, _c_i64, _c_i64,                  # E, N, K
        _p, _c_int, _c_i64, _p]),                # y, y_dtype, ldy, stream
    "ep_expert_matmul_grouped_workspace": (_sz, [_c_i64, _c_i64, _c_i64]),
    "ep_expert_matmul_grouped": (_c_int, [
        _p, _c_int, _c_i64, _p, _c_i64,         # x, x_dtype, ldx, expert_ids (int32), T
        _p, _p, _c_int, _c_i64,                  # packed, scale, scale_dtype, ld_scale
        _p, _c_int, _c_int, _c_int,              # cb, cb_dtype, levels, group
        _c_i64, _c_i64, _c_i64,                  # E, N, K
        _p, _c_int, _c_i64,                      # y, y_dtype, ldy
        _p, _sz, _p]),                           # workspace, bytes, stream
    "ep_dequant_matmul_bwd_workspace": (_sz, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "ep_dequant_matmul_bwd": (_c_int, [
        _p, _c_int, _c_i64,                      # gy, gy_dtype, ldgy
        _p, _c_int, _c_i64,                      # x, x_dtype, ldx
        _p, _p, _c_int, _c_i64,                  # packed, scale, scale_dtype, ld_scale
        _p, _c_int, _c_int, _c_int,              # cb, cb_dtype, levels, group
        _c_i64, _c_i64, _c_i64,                  # M, N, K
        _p, _c_int, _c_i64,                      # grad_x, gx_dtype, ldgx
        _p, _p, _c_i64,                          # grad_cb, grad_scale, ld_gscale
        _p, _sz, _p]),                           # workspace, bytes, stream
    "ep_unpack_indices": (_c_int, [_p, _c_i64, _c_int, _p, _p]),
    "ep_dequant_tile": (_c_int, [
        _p, _p, _c_int, _c_i64, _p, _c_int, _c_int, _c_int, _c_i64, _c_i64,
        _p, _c_int, _c_i64, _p]),
    "ep_embedding_rows": (_c_int, [
        _p, _p, _c_int, _c_i64, _p, _c_int, _c_int, _c_int, _c_i64, _c_i64,
        _p, _c_i64, _p, _c_int, _c_i64, _p]),
    # include/epure_decode.h
    "ep_fused_gemv": (_c_int, [
        _c_int, _p, _c_int, _p, ctypes.c_float,  # xsrc, x, x_dtype, x_aux, eps
        _c_i64, _c_int, _c_int, _c_int, _c_int,  # K, group, levels, scale_dtype, cb_dtype
        _c_int, _p, _p, _p, _p, _p,              # nseg, packed[], scale[], cb[], y[], N[]
        _c_int, _c_int, _p]),                    # y_dtype, accumulate, stream
    "ep_attention_workspace": (_sz, [_c_int, _c_int, _c_int]),
    "ep_decode_attention": (_c_int, [
        _p, _p, _p, _p, _p, ctypes.c_float,      # q, k, v, qn_w, kn_w, qk_eps
        _p, _p, _p, _p, _p, _p, _p, _p,          # kcache, vcache, cos, sin, state, part, ctr, out
        _c_int, _c_int, _c_int, _c_int, ctypes.c_float, _p]),
    "ep_lm_head_argmax": (_c_int, [
        _p, _p, ctypes.c_float, _p, _p, _c_int, _c_int,   # h, norm_w, eps, W, logits, V, H
        _p, _p, _p, _p, _p, _c_int, _p, _p, _p,           # part_val, part_idx, counter, state,
        _c_int, _c_int, _p]),                             # prompt, n_prompt, tokens, argmax,
                                                          # embed, max_pos, grid, stream
    "ep_embed_token": (_c_int, [_p, _p, _p, _c_int, _p]),
    "ep_decode_step_layer_bytes": (_sz, []),
    "ep_decode_step_workspace": (_sz, [_c_int] * 6),
    "ep_decode_step_serves": (_c_int, [_c_int] * 10),
    "ep_decode_step": (_c_int, [
        _p, _c_int, _p, _p, _sz,                 # layers, n_layers, h, workspace, bytes
        _p, _p, _p,                              # cos, sin, state
        _c_int, _c_int, _c_int, _c_int, _c_int,  # H, I, Hq, Hkv, D
        _c_int, _c_int, _c_int, _c_int, _c_int,  # max_pos, levels, group, scale_dtype, cb_dtype
        ctypes.c_float, ctypes.c_float, ctypes.c_float,  # eps, qk_eps, att_scale
        _p, _p]),                                # trace, stream
}

XSRC_PLAIN, XSRC_RMSNORM, XSRC_SWIGLU = 0, 1, 2

lib = None
LOAD_ERROR = None


def _load():
    global lib, LOAD_ERROR
    if lib is not None or LOAD_ERROR is not None:
        return lib
    try:
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.ep_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_NAME} ABI {handle.ep_abi_version()} != {ABI_VERSION}")
        lib = handle
    except Exception as exc:                    # noqa: BLE001 - recorded and re-raised by callers
        LOAD_ERROR = exc
    return lib


def dtype_code(dt):
    return _DT.get(dt)


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def last_error():
    msg = lib.ep_last_error() if lib is not None else b""
    return msg.decode(errors="replace") if msg else ""


def check(rc, what):
    """Map a C ABI return code: 0 -> True, > 0 (decline) -> False, < 0 -> raise."""
    if rc == OK:
        return True
    if rc > 0:
        return False
    raise RuntimeError(f"{what} failed ({rc}): {last_error()}")
