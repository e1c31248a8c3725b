"""ctypes binding of libwsl.so (the C ABI declared in include/wsl_lora.h).

torch is imported first so that the process-wide HIP runtime is the one PyTorch-ROCm
ships; libwsl then binds to that same runtime. There is no fallback: if the library is
missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime libwsl links against)

# WSL_LIB names another build of the same library (the instrumented libwsl_stamps.so that
# `bench.py --only stamps` reads); by default the in-tree libwsl.so.
LIB_PATH = os.environ.get("WSL_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwsl.so")

WSL_OK = 0
WSL_E_INVALID_ARG = -1
WSL_E_SHAPE = -2
WSL_E_DTYPE = -3
WSL_E_ALIGN = -4
WSL_E_WORKSPACE = -5
WSL_E_DEVICE = -6
WSL_E_LAUNCH = -7

WSL_FUSE_RMSNORM = 1
WSL_FUSE_SWIGLU = 2
WSL_FUSE_RESIDUAL = 4

WSL_DTYPE_BF16 = 0
WSL_DTYPE_FP8_E4M3 = 1
WSL_DTYPE_FP8_E4M3_ACT8 = 2
WSL_MAX_RANK = 256
WSL_NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024

# Every symbol include/wsl_lora.h and include/wsl_decode.h declare.
EXPORTED = (
    "wsl_lora_linear_workspace_bytes",
    "wsl_lora_linear_fwd",
    "wsl_lora_linear_fwd_noalloc",
    "wsl_lora_linear_grouped_workspace_bytes",
    "wsl_lora_linear_grouped_fwd",
    "wsl_lora_linear_bcast_workspace_bytes",
    "wsl_lora_linear_bcast_fwd",
    "wsl_lora_linear_bwd_weights_supported",
    "wsl_lora_linear_bwd_weights_workspace_bytes",
    "wsl_lora_linear_bwd_weights",
    "wsl_lora_linear_bwd_input_supported",
    "wsl_lora_linear_bwd_input_workspace_bytes",
    "wsl_lora_linear_bwd_input",
    "wsl_factorized_embedding_fwd",
    "wsl_last_error",
    "wsl_version",
    "wsl_set_option",
    "wsl_get_option",
    "wsl_lora_linear_plan",
    "wsl_rmsnorm_fwd",
    "wsl_qk_norm_rope_fwd",
    "wsl_decode_attention_workspace_bytes",
    "wsl_decode_attention_fwd",
    "wsl_decode_attention_step_workspace_bytes",
    "wsl_decode_attention_step_fwd",
    "wsl_swiglu_fwd",
    "wsl_argmax_rows_fwd",
    "wsl_argmax_rows_workspace_bytes",
    "wsl_lora_linear_fused_supported",
    "wsl_lora_linear_fused_fwd",
    "wsl_decode_last_error",
    "wsl_tied_head_argmax_workspace_bytes",
    "wsl_tied_head_argmax_supported",
    "wsl_tied_head_argmax_fwd",
    "wsl_lora_linear_chain_supported",
    "wsl_lora_linear_chain_workspace_bytes",
    "wsl_lora_linear_chain_fwd",
    "wsl_lora_linear_chain_status",
)

WSL_CHAIN_MAX_STAGES = 8


class ChainStage(ctypes.Structure):
    """wsl_chain_stage (include/wsl_decode.h)."""
    _fields_ = [("x", ctypes.c_void_p), ("ldx", ctypes.c_int64), ("norm_w", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("w", ctypes.c_void_p), ("ldw", ctypes.c_int64), ("a", ctypes.c_void_p), ("lda", ctypes.c_int64),
                ("b", ctypes.c_void_p), ("ldb", ctypes.c_int64), ("scale", ctypes.c_float),
                ("residual", ctypes.c_void_p), ("ldr", ctypes.c_int64), ("y", ctypes.c_void_p),
                ("ldy", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("r", ctypes.c_int64),
                ("fuse", ctypes.c_int32), ("n_groups", ctypes.c_int32), ("group_n", ctypes.c_int64 * 4),
                ("after_previous", ctypes.c_int32)]

_lib = None
_lock = threading.Lock()

_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p


class WSLError(RuntimeError):
    """A libwsl call failed on the device side (workspace, device, launch)."""


# Path overrides (WSL_OPT_* in include/wsl_lora.h) by name; 0 is the library's own choice.
OPTIONS = {
    "prefill_strips": 1,     # -1: one output tile per workgroup
    "prefill_split": 2,      # -1: no split-K inside a launch; 2..16: that split count
    "prefill_medium": 3,     # -1: never the medium-M split form
    "fp8_prefill": 4,        # 0: by launch width; 1: fp8 W decoded onto the bf16 matrix cores; 2: fp8 matrix cores
    "decode_passes": 5,      # -1: K splits only; 1: passes wherever the slices allow
    "decode_wide": 6,        # 1: 65-72 tokens on the decode path's wide form
    "decode_spin_limit": 7,  # n > 0: poll bound of the decode hand-offs; -1: no polling
    "decode_res_splits": 8,  # 2..8: K splits of the decode step's residual-epilogue launches
    "prefill_shared_t": 9,   # -1: T in every tile; 1: shared T, every tile on the no-wait path; 2: at any K
}

# wsl_plan_info.path values
PATHS = {0: "none", 1: "prefill", 2: "prefill_splitk", 3: "prefill_medium", 4: "prefill_fp8", 5: "decode",
         6: "generic"}


class PlanInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("path", "launches", "tile_m", "tile_n", "rank_blocks",
                                               "rank_prepass", "strip_tiles", "k_splits", "workgroups",
                                               "shared_t")]


def _declare(lib: ctypes.CDLL) -> None:
    lib.wsl_version.restype = ctypes.c_int
    lib.wsl_version.argtypes = []
    lib.wsl_set_option.restype = ctypes.c_int
    lib.wsl_set_option.argtypes = [ctypes.c_int32, _c_i64]
    lib.wsl_get_option.restype = ctypes.c_int
    lib.wsl_get_option.argtypes = [ctypes.c_int32, ctypes.POINTER(_c_i64)]
    lib.wsl_lora_linear_plan.restype = ctypes.c_int
    lib.wsl_lora_linear_plan.argtypes = [_c_i64, _c_i64, _c_i64, ctypes.c_int32, ctypes.POINTER(_c_i64),
                                         ctypes.c_int32, ctypes.POINTER(PlanInfo)]
    lib.wsl_last_error.restype = ctypes.c_char_p
    lib.wsl_last_error.argtypes = []
    lib.wsl_lora_linear_workspace_bytes.restype = ctypes.c_int
    lib.wsl_lora_linear_workspace_bytes.argtypes = [
        _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]
    lib.wsl_lora_linear_fwd.restype = ctypes.c_int
    lib.wsl_lora_linear_fwd.argtypes = [
        _c_vp, _c_i64,                   # x, ldx
        _c_vp, _c_i64, ctypes.c_int32, _c_vp,  # w, ldw, w_dtype, w_scale
        _c_vp, _c_i64,                   # a, lda
        _c_vp, _c_i64,                   # b, ldb
        ctypes.c_float,                  # scale
        _c_vp, _c_i64,                   # y, ldy
        _c_i64, _c_i64, _c_i64, _c_i64,  # M, N, K, r
        _c_vp, ctypes.c_size_t,          # workspace, bytes
        _c_vp,                           # stream
    ]
    lib.wsl_lora_linear_fwd_noalloc.restype = ctypes.c_int
    lib.wsl_lora_linear_fwd_noalloc.argtypes = [
        _c_vp, _c_i64,                   # x, ldx
        _c_vp, _c_i64, ctypes.c_int32, _c_vp,  # w, ldw, w_dtype, w_scale
        _c_vp, _c_i64,                   # a, lda
        _c_vp, _c_i64,                   # b, ldb
        ctypes.c_float,                  # scale
        _c_vp, _c_i64,                   # y, ldy
        _c_i64, _c_i64, _c_i64, _c_i64,  # M, N, K, r
        _c_vp,                           # stream
    ]
    lib.wsl_lora_linear_grouped_workspace_bytes.restype = ctypes.c_int
    lib.wsl_lora_linear_grouped_workspace_bytes.argtypes = [
        _c_i64, _c_i64, _c_i64, ctypes.c_int32, ctypes.POINTER(_c_i64), ctypes.c_int32,
        ctypes.POINTER(ctypes.c_size_t)]
    lib.wsl_lora_linear_grouped_fwd.restype = ctypes.c_int
    lib.wsl_lora_linear_grouped_fwd.argtypes = [
        _c_vp, _c_i64,                   # x, ldx
        _c_vp, _c_i64, ctypes.c_int32, _c_vp,  # w, ldw, w_dtype, w_scale
        _c_vp, _c_i64,                   # a, lda
        _c_vp, _c_i64,                   # b, ldb
        ctypes.c_float,                  # scale
        _c_vp, _c_i64,                   # y, ldy
        _c_i64, _c_i64, _c_i64,          # M, K, r
        ctypes.c_int32, ctypes.POINTER(_c_i64),  # n_groups, group_n
        _c_vp, ctypes.c_size_t,          # workspace, bytes
        _c_vp,                           # stream
    ]
    lib.wsl_lora_linear_bcast_workspace_bytes.restype = ctypes.c_int
    lib.wsl_lora_linear_bcast_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int32,
                                                          ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]
    lib.wsl_lora_linear_bcast_fwd.restype = ctypes.c_int
    lib.wsl_lora_linear_bcast_fwd.argtypes = [
        _c_vp, _c_i64,                   # x, ldx
        _c_vp, _c_i64, ctypes.c_int32, _c_vp,  # w, ldw, w_dtype, w_scale
        _c_vp, _c_i64,                   # a, lda
        _c_vp, _c_i64,                   # b, ldb
        ctypes.c_float,                  # scale
        _c_vp, _c_i64,                   # y, ldy
        _c_i64, _c_i64, _c_i64, _c_i64,  # M, N, K, r
        _c_i64, _c_i64, ctypes.c_int32,  # base_n, g, n_groups
        _c_vp, ctypes.c_size_t,          # workspace, bytes
        _c_vp,                           # stream
    ]
    lib.wsl_lora_linear_bwd_weights_supported.restype = ctypes.c_int
    lib.wsl_lora_linear_bwd_weights_supported.argtypes = [
        _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,  # x, ldx, gy, ldg, a, lda, b, ldb
        _c_i64, _c_i64, _c_i64, _c_i64]                              # M, N, K, r
    lib.wsl_lora_linear_bwd_weights_workspace_bytes.restype = ctypes.c_int
    lib.wsl_lora_linear_bwd_weights_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64,
                                                                ctypes.POINTER(ctypes.c_size_t)]
    lib.wsl_lora_linear_bwd_weights.restype = ctypes.c_int
    lib.wsl_lora_linear_bwd_weights.argtypes = [
        _c_vp, _c_i64, _c_vp, _c_i64,    # x, ldx, gy, ldg
        _c_vp, _c_i64, _c_vp, _c_i64,    # a, lda, b, ldb
        ctypes.c_float,                  # scale
        _c_i64, _c_i64, _c_i64, _c_i64,  # M, N, K, r
        _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,  # dw, lddw, da, ldda, db, lddb
        _c_vp, ctypes.c_size_t,          # workspace, bytes
        _c_vp,                           # stream
    ]
    lib.wsl_lora_linear_bwd_input_supported.restype = ctypes.c_int
    lib.wsl_lora_linear_bwd_input_supported.argtypes = [
        _c_vp, _c_i64, _c_vp, _c_i64,    # gy, ldg, w, ldw
        ctypes.c_int32, _c_vp,           # w_dtype, w_scale
        _c_vp, _c_i64, _c_vp, _c_i64,    # a, lda, b, ldb
        _c_vp, _c_i64,                   # dx, lddx
        _c_i64, _c_i64, _c_i64, _c_i64]  # M, N, K, r
    lib.wsl_lora_linear_bwd_input_workspace_bytes.restype = ctypes.c_int
    lib.wsl_lora_linear_bwd_input_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64,
                                                              ctypes.POINTER(ctypes.c_size_t)]
    lib.wsl_lora_linear_bwd_input.restype = ctypes.c_int
    lib.wsl_lora_linear_bwd_input.argtypes = [
        _c_vp, _c_i64, _c_vp, _c_i64,    # gy, ldg, w, ldw
        ctypes.c_int32, _c_vp,           # w_dtype, w_scale
        _c_vp, _c_i64, _c_vp, _c_i64,    # a, lda, b, ldb
        ctypes.c_float,                  # scale
        _c_vp, _c_i64,                   # dx, lddx
        _c_i64, _c_i64, _c_i64, _c_i64,  # M, N, K, r
        _c_vp, ctypes.c_size_t,          # workspace, bytes
        _c_vp,                           # stream
    ]
    lib.wsl_decode_last_error.restype = ctypes.c_char_p
    lib.wsl_decode_last_error.argtypes = []
    lib.wsl_rmsnorm_fwd.restype = ctypes.c_int
    lib.wsl_rmsnorm_fwd.argtypes = [
        _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, ctypes.c_float,  # x, ldx, residual, ldr, weight, eps
        _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]   # out, ldo, h_out, ldh, rows, dim, stream
    lib.wsl_qk_norm_rope_fwd.restype = ctypes.c_int
    lib.wsl_qk_norm_rope_fwd.argtypes = [
        _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,        # qkv, ldqkv, batch, n_heads, n_kv, head_dim
        _c_vp, _c_vp, ctypes.c_float, _c_vp, _c_vp,          # q_norm_w, k_norm_w, eps, rope, pos
        _c_vp, _c_vp, _c_vp, _c_i64, _c_vp]                  # q_out, k_cache, v_cache, cache_len, stream
    lib.wsl_decode_attention_workspace_bytes.restype = ctypes.c_size_t
    lib.wsl_decode_attention_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]
    lib.wsl_decode_attention_fwd.restype = ctypes.c_int
    lib.wsl_decode_attention_fwd.argtypes = [
        _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,  # q, k, v, batch, nh, nkv, hd, cache_len
        _c_vp, ctypes.c_float, _c_vp, _c_vp, ctypes.c_size_t, _c_vp]  # pos, scale, out, workspace, bytes, stream
    lib.wsl_decode_attention_step_workspace_bytes.restype = ctypes.c_size_t
    lib.wsl_decode_attention_step_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]
    lib.wsl_decode_attention_step_fwd.restype = ctypes.c_int
    lib.wsl_decode_attention_step_fwd.argtypes = [
        _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,        # qkv, ldqkv, batch, n_heads, n_kv, head_dim
        _c_vp, _c_vp, ctypes.c_float, _c_vp, _c_vp,          # q_norm_w, k_norm_w, eps, rope, pos
        _c_vp, _c_vp, _c_i64, ctypes.c_float, _c_vp,         # k_cache, v_cache, cache_len, scale, out
        _c_vp, ctypes.c_size_t, _c_vp]                       # workspace, bytes, stream
    lib.wsl_swiglu_fwd.restype = ctypes.c_int
    lib.wsl_swiglu_fwd.argtypes = [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp]
    lib.wsl_lora_linear_fused_supported.restype = ctypes.c_int
    lib.wsl_lora_linear_fused_supported.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int32]
    lib.wsl_lora_linear_fused_fwd.restype = ctypes.c_int
    lib.wsl_lora_linear_fused_fwd.argtypes = [
        _c_vp, _c_i64, _c_vp, ctypes.c_float, _c_vp, _c_i64,  # x, ldx, norm_w, eps, w, ldw
        _c_vp, _c_i64, _c_vp, _c_i64, ctypes.c_float,          # a, lda, b, ldb, scale
        _c_vp, _c_i64, _c_vp, _c_i64,                          # residual, ldr, y, ldy
        _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int32,        # M, N, K, r, fuse
        _c_vp, ctypes.c_size_t, _c_vp]                         # workspace, bytes, stream
    chain_p = ctypes.POINTER(ChainStage)
    lib.wsl_lora_linear_chain_supported.restype = ctypes.c_int
    lib.wsl_lora_linear_chain_supported.argtypes = [_c_i64, ctypes.c_int32, chain_p]
    lib.wsl_lora_linear_chain_workspace_bytes.restype = ctypes.c_int
    lib.wsl_lora_linear_chain_workspace_bytes.argtypes = [_c_i64, ctypes.c_int32, chain_p,
                                                          ctypes.POINTER(ctypes.c_size_t)]
    lib.wsl_lora_linear_chain_fwd.restype = ctypes.c_int
    lib.wsl_lora_linear_chain_fwd.argtypes = [_c_i64, ctypes.c_int32, chain_p, _c_vp, ctypes.c_size_t, _c_vp]
    lib.wsl_lora_linear_chain_status.restype = ctypes.c_int
    lib.wsl_lora_linear_chain_status.argtypes = [_c_vp, _c_vp, ctypes.POINTER(ctypes.c_int32)]
    lib.wsl_tied_head_argmax_workspace_bytes.restype = ctypes.c_size_t
    lib.wsl_tied_head_argmax_workspace_bytes.argtypes = [_c_i64]
    lib.wsl_tied_head_argmax_supported.restype = ctypes.c_int
    lib.wsl_tied_head_argmax_supported.argtypes = [_c_i64, _c_i64, _c_i64]
    lib.wsl_tied_head_argmax_fwd.restype = ctypes.c_int
    lib.wsl_tied_head_argmax_fwd.argtypes = [
        _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,  # x, ldx, w, ldw, N, K, M
        _c_vp, _c_vp, ctypes.c_size_t, _c_vp]                  # out, workspace, bytes, stream
    lib.wsl_argmax_rows_fwd.restype = ctypes.c_int
    lib.wsl_argmax_rows_fwd.argtypes = [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, ctypes.c_size_t, _c_vp]
    lib.wsl_argmax_rows_workspace_bytes.restype = ctypes.c_size_t
    lib.wsl_argmax_rows_workspace_bytes.argtypes = [_c_i64, _c_i64]
    lib.wsl_factorized_embedding_fwd.restype = ctypes.c_int
    lib.wsl_factorized_embedding_fwd.argtypes = [
        _c_vp, _c_i64,                   # ids, n_ids
        _c_vp, _c_i64, _c_i64, _c_i64,   # emb, lde, vocab, k
        _c_vp, _c_i64, _c_i64,           # proj, ldp, hidden
        _c_vp, _c_i64,                   # out, ldo
        _c_vp,                           # stream
    ]


def lib() -> ctypes.CDLL:
    """Returns the loaded library, loading it on first use. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libwsl.so not found at {LIB_PATH}; build it with "
                    "`python -m weightshared_torchtitan_amd.build` (hipcc, gfx950)")
            handle = ctypes.CDLL(LIB_PATH)
            _declare(handle)
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().wsl_last_error().decode("utf-8", "replace")


def decode_last_error() -> str:
    return lib().wsl_decode_last_error().decode("utf-8", "replace")


def check(rc: int, what: str, decode: bool = False) -> None:
    """Maps a WSL_E_* code to the matching Python exception (decode=True: the error text of
    the decode-step entry points)."""
    if rc == WSL_OK:
        return
    msg = f"{what}: {decode_last_error() if decode else last_error()} (code {rc})"
    if rc in (WSL_E_INVALID_ARG, WSL_E_SHAPE, WSL_E_ALIGN):
        raise ValueError(msg)
    if rc == WSL_E_DTYPE:
        raise TypeError(msg)
    raise WSLError(msg)


def workspace_bytes(M: int, N: int, K: int, r: int, w_dtype: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib().wsl_lora_linear_workspace_bytes(M, N, K, r, w_dtype, ctypes.byref(out)),
          "wsl_lora_linear_workspace_bytes")
    return int(out.value)


WSL_MAX_GROUPS = 4


def group_array(group_n) -> "ctypes.Array":
    """The host array of group widths a grouped call takes."""
    return (_c_i64 * len(group_n))(*[int(n) for n in group_n])


def bcast_workspace_bytes(M: int, N: int, K: int, r: int, n_groups: int, w_dtype: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib().wsl_lora_linear_bcast_workspace_bytes(M, N, K, r, n_groups, w_dtype, ctypes.byref(out)),
          "wsl_lora_linear_bcast_workspace_bytes")
    return int(out.value)


def grouped_workspace_bytes(M: int, K: int, r: int, group_n, w_dtype: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib().wsl_lora_linear_grouped_workspace_bytes(M, K, r, len(group_n), group_array(group_n), w_dtype,
                                                        ctypes.byref(out)),
          "wsl_lora_linear_grouped_workspace_bytes")
    return int(out.value)


def bwd_input_workspace_bytes(M: int, N: int, K: int, r: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib().wsl_lora_linear_bwd_input_workspace_bytes(M, N, K, r, ctypes.byref(out)),
          "wsl_lora_linear_bwd_input_workspace_bytes")
    return int(out.value)


def bwd_weights_workspace_bytes(M: int, N: int, K: int, r: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib().wsl_lora_linear_bwd_weights_workspace_bytes(M, N, K, r, ctypes.byref(out)),
          "wsl_lora_linear_bwd_weights_workspace_bytes")
    return int(out.value)


def set_option(name: str, value: int) -> None:
    """Sets a path override (see OPTIONS); 0 restores the library's own choice."""
    check(lib().wsl_set_option(OPTIONS[name], int(value)), f"wsl_set_option({name})")


def get_option(name: str) -> int:
    out = _c_i64(0)
    check(lib().wsl_get_option(OPTIONS[name], ctypes.byref(out)), f"wsl_get_option({name})")
    return int(out.value)


def plan(M: int, K: int, r: int, group_n, w_dtype: int = WSL_DTYPE_BF16) -> dict:
    """The plan a call of these sizes takes (dense, aligned operands): a dict of the
    wsl_plan_info fields, with `path` by name."""
    info = PlanInfo()
    check(lib().wsl_lora_linear_plan(M, K, r, len(group_n), group_array(group_n), w_dtype, ctypes.byref(info)),
          "wsl_lora_linear_plan")
    out = {n: int(getattr(info, n)) for n, _ in PlanInfo._fields_}
    out["path"] = PATHS[out["path"]]
    return out
