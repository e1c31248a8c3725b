"""The C ABI without a GPU: libwsl.so loads, exports every symbol include/wsl_lora.h
declares, and rejects bad arguments with the documented WSL_E_* codes before it touches
a device. No call here launches a kernel; pointers passed are never dereferenced on the
host (validation fails first)."""
import ctypes
import os
import re

import pytest

from weightshared_torchtitan_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wsl_lora.h")
HEADERS = sorted(os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))
                 if f.endswith(".h"))

needs_lib = pytest.mark.skipif(not os.path.exists(N.LIB_PATH),
                               reason="libwsl.so not built (run __graft_entry__.build())")


def _header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(wsl_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def _header_defines():
    out = {}
    for name, val in re.findall(r"#define\s+(WSL_[A-Z0-9_]+)\s+\(?(-?\d+)\)?", open(HEADER).read()):
        out[name] = int(val)
    return out


def test_binding_lists_every_header_function():
    assert sorted(N.EXPORTED) == _header_functions()


def test_python_constants_match_header():
    d = _header_defines()
    for name in ("WSL_OK", "WSL_E_INVALID_ARG", "WSL_E_SHAPE", "WSL_E_DTYPE", "WSL_E_ALIGN",
                 "WSL_E_WORKSPACE", "WSL_E_DEVICE", "WSL_E_LAUNCH", "WSL_DTYPE_BF16",
                 "WSL_DTYPE_FP8_E4M3", "WSL_MAX_RANK"):
        assert getattr(N, name) == d[name], name


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(N.LIB_PATH)
    for name in _header_functions():
        assert hasattr(lib, name), name


@needs_lib
def test_version_and_empty_error():
    lib = N.lib()
    assert lib.wsl_version() == 101
    sz = ctypes.c_size_t()
    assert lib.wsl_lora_linear_workspace_bytes(16, 64, 64, 8, 0, ctypes.byref(sz)) == N.WSL_OK
    assert N.last_error() == ""


@needs_lib
@pytest.mark.parametrize("M,Nn,K,r,dt,code", [
    (-1, 64, 64, 8, 0, N.WSL_E_SHAPE),
    (4, 0, 64, 8, 0, N.WSL_E_SHAPE),
    (4, 64, 0, 8, 0, N.WSL_E_SHAPE),
    (4, 64, 64, -1, 0, N.WSL_E_SHAPE),
    (4, 64, 64, 257, 0, N.WSL_E_SHAPE),
    (4, 64, 64, 8, 7, N.WSL_E_DTYPE),
])
def test_workspace_query_rejects_bad_sizes(M, Nn, K, r, dt, code):
    sz = ctypes.c_size_t()
    assert N.lib().wsl_lora_linear_workspace_bytes(M, Nn, K, r, dt, ctypes.byref(sz)) == code
    assert N.last_error() != ""


@needs_lib
def test_workspace_query_null_out_pointer():
    assert N.lib().wsl_lora_linear_workspace_bytes(4, 64, 64, 8, 0, None) == N.WSL_E_INVALID_ARG


@needs_lib
@pytest.mark.parametrize("M", [1, 8, 64, 65, 8192])
def test_workspace_includes_counter_prefix(M):
    # Every path's scratch sits after the WSL_COUNTER_BYTES prefix.
    b = N.workspace_bytes(M, 2048, 2048, 64, N.WSL_DTYPE_BF16)
    assert b >= _header_defines()["WSL_COUNTER_BYTES"]
    # r > 64 on the prefill path materialises T [M, r] bf16
    big = N.workspace_bytes(M, 2048, 2048, 128, N.WSL_DTYPE_BF16)
    assert big >= b


@needs_lib
def test_workspace_holds_split_prepass_partials():
    # M = 4096, K = 4096, r = 128: 32 rank tiles, so the pre-pass splits K 8 ways and
    # keeps 8 fp32 partial slices [M, r] beside T [M, r] bf16.
    M, K, r = 4096, 4096, 128
    need = N.workspace_bytes(M, 1024, K, r, N.WSL_DTYPE_BF16)
    assert need >= _header_defines()["WSL_COUNTER_BYTES"] + M * r * 2 + 8 * M * r * 4
    # one K tile cannot be split: T only
    small = N.workspace_bytes(M, 1024, 64, r, N.WSL_DTYPE_BF16)
    assert small < _header_defines()["WSL_COUNTER_BYTES"] + M * r * 2 + M * r * 4


P = 0x100000  # a 256-aligned fake device address; never dereferenced


def _fwd(**kw):
    a = dict(x=P, ldx=64, w=P, ldw=64, w_dtype=0, w_scale=None, a=P, lda=64, b=P, ldb=8,
             scale=2.0, y=P, ldy=64, M=4, N=64, K=64, r=8, ws=P, ws_bytes=1 << 24, stream=None)
    a.update(kw)
    return N.lib().wsl_lora_linear_fwd(a["x"], a["ldx"], a["w"], a["ldw"], a["w_dtype"], a["w_scale"],
                                       a["a"], a["lda"], a["b"], a["ldb"], a["scale"], a["y"], a["ldy"],
                                       a["M"], a["N"], a["K"], a["r"], a["ws"], a["ws_bytes"], a["stream"])


@needs_lib
@pytest.mark.parametrize("kw,code", [
    (dict(x=None), N.WSL_E_INVALID_ARG),
    (dict(y=None), N.WSL_E_INVALID_ARG),
    (dict(w=None, r=0), N.WSL_E_INVALID_ARG),
    (dict(a=None), N.WSL_E_INVALID_ARG),
    (dict(w_dtype=1), N.WSL_E_INVALID_ARG),          # fp8 without w_scale
    (dict(w_scale=P), N.WSL_E_INVALID_ARG),          # w_scale with bf16 w
    (dict(ldx=63), N.WSL_E_SHAPE),
    (dict(ldw=63), N.WSL_E_SHAPE),
    (dict(lda=63), N.WSL_E_SHAPE),
    (dict(ldb=7), N.WSL_E_SHAPE),
    (dict(ldy=63), N.WSL_E_SHAPE),
    (dict(r=300), N.WSL_E_SHAPE),
    (dict(w_dtype=5), N.WSL_E_DTYPE),
    (dict(x=P + 1), N.WSL_E_ALIGN),
    (dict(y=P + 1), N.WSL_E_ALIGN),
    (dict(ws=None), N.WSL_E_WORKSPACE),
    (dict(ws_bytes=16), N.WSL_E_WORKSPACE),
    (dict(ws=P + 128), N.WSL_E_ALIGN),
])
def test_fwd_validation_codes(kw, code):
    assert _fwd(**kw) == code
    assert N.last_error() != ""


@needs_lib
def test_fwd_empty_batch_is_a_no_op():
    assert _fwd(M=0, x=None, y=None, ws=None, ws_bytes=0) == N.WSL_OK


@needs_lib
def test_embedding_validation_codes():
    lib = N.lib()
    ok = dict(ids=P, n=4, emb=P, lde=16, V=100, k=16, proj=P, ldp=16, H=32, out=P, ldo=32)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return lib.wsl_factorized_embedding_fwd(a["ids"], a["n"], a["emb"], a["lde"], a["V"], a["k"],
                                                a["proj"], a["ldp"], a["H"], a["out"], a["ldo"], None)

    assert call(n=-1) == N.WSL_E_SHAPE
    assert call(k=2048) == N.WSL_E_SHAPE
    assert call(lde=8) == N.WSL_E_SHAPE
    assert call(ids=None) == N.WSL_E_INVALID_ARG
    assert call(ids=P + 4) == N.WSL_E_ALIGN
    assert call(n=0, ids=None) == N.WSL_OK


def test_python_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        N.check(N.WSL_E_SHAPE, "x")
    with pytest.raises(TypeError):
        N.check(N.WSL_E_DTYPE, "x")
    with pytest.raises(N.WSLError):
        N.check(N.WSL_E_LAUNCH, "x")
    N.check(N.WSL_OK, "x")


def test_ops_refuse_cpu_tensors():
    # No CPU fallback: the product path raises on host tensors.
    import torch

    from weightshared_torchtitan_amd import ops
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w = torch.zeros(32, 64, dtype=torch.bfloat16)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops.lora_linear(x, w)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops.factorized_embedding(torch.zeros(3, dtype=torch.int64), torch.zeros(10, 8, dtype=torch.bfloat16),
                                 torch.zeros(16, 8, dtype=torch.bfloat16))
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops.lora_linear_grouped(x, [w, w], [torch.zeros(8, 64, dtype=torch.bfloat16)] * 2,
                                [torch.zeros(32, 8, dtype=torch.bfloat16)] * 2, 2.0)


def test_grouped_op_fake_kernel_shapes():
    # the meta implementation gives [..., sum of widths] bf16, as the device op does
    import torch

    from weightshared_torchtitan_amd import ops
    with torch.device("meta"):
        x = torch.empty(3, 5, 64, dtype=torch.bfloat16)
        w = torch.empty(96, 64, dtype=torch.bfloat16)
        a = torch.empty(3 * 8, 64, dtype=torch.bfloat16)
        b = torch.empty(96, 8, dtype=torch.bfloat16)
        y = ops.lora_linear_grouped_op(x, w, None, a, b, 2.0, [64, 16, 16])
    assert y.shape == (3, 5, 96) and y.dtype == torch.bfloat16 and y.device.type == "meta"


def test_weight_grads_op_fake_kernel_shapes():
    # the meta implementation gives dW [N, K], dA [r, K], dB [N, r] bf16 and an empty tensor
    # for each gradient not asked for, as the device op does
    import torch

    from weightshared_torchtitan_amd import ops
    with torch.device("meta"):
        x = torch.empty(40, 64, dtype=torch.bfloat16)
        gy = torch.empty(40, 128, dtype=torch.bfloat16)
        a = torch.empty(8, 64, dtype=torch.bfloat16)
        b = torch.empty(128, 8, dtype=torch.bfloat16)
        dw, da, db = ops.lora_linear_weight_grads_op(x, gy, a, b, 2.0, True, True, True)
        none = ops.lora_linear_weight_grads_op(x, gy, a, b, 2.0, True, False, False)
    assert (dw.shape, da.shape, db.shape) == ((128, 64), (8, 64), (128, 8))
    assert all(t.dtype == torch.bfloat16 and t.device.type == "meta" for t in (dw, da, db))
    assert none[0].shape == (128, 64) and none[1].numel() == 0 and none[2].numel() == 0


@needs_lib
def test_decode_step_validation_codes():
    lib = N.lib()
    P2 = P
    # rmsnorm: dim not a multiple of 8; misaligned pointer; empty batch
    assert lib.wsl_rmsnorm_fwd(P2, 64, None, 0, P2, 1e-6, P2, 64, None, 0, 4, 60, None) == N.WSL_E_SHAPE
    assert lib.wsl_rmsnorm_fwd(P2 + 2, 64, None, 0, P2, 1e-6, P2, 64, None, 0, 4, 64, None) == N.WSL_E_ALIGN
    assert lib.wsl_rmsnorm_fwd(None, 64, None, 0, None, 1e-6, None, 64, None, 0, 0, 64, None) == N.WSL_OK
    assert N.decode_last_error() == ""
    # qk norm + rope: unsupported head_dim; ld too small
    assert lib.wsl_qk_norm_rope_fwd(P2, 4096, 2, 16, 8, 96, P2, P2, 1e-6, P2, P2, P2, P2, P2, 64, None) == N.WSL_E_SHAPE
    assert lib.wsl_qk_norm_rope_fwd(P2, 100, 2, 16, 8, 128, P2, P2, 1e-6, P2, P2, P2, P2, P2, 64, None) == N.WSL_E_SHAPE
    assert N.decode_last_error() != ""
    # attention: heads not a multiple of kv heads / unsupported grouping
    assert lib.wsl_decode_attention_fwd(P2, P2, P2, 2, 12, 8, 128, 64, P2, 0.1, P2, P2, 1 << 20, None) == N.WSL_E_SHAPE
    assert lib.wsl_decode_attention_fwd(P2, P2, P2, 2, 48, 3, 128, 64, P2, 0.1, P2, P2, 1 << 20, None) == N.WSL_E_SHAPE
    need = lib.wsl_decode_attention_workspace_bytes(8, 16, 8, 128, 1024)
    assert need == 8 * 16 * 16 * 130 * 4
    assert lib.wsl_decode_attention_fwd(P2, P2, P2, 8, 16, 8, 128, 1024, P2, 0.1, P2, P2, need - 4, None) \
        == N.WSL_E_WORKSPACE
    # swiglu: ld below 2 * ffn
    assert lib.wsl_swiglu_fwd(P2, 100, 4, 64, P2, 64, None) == N.WSL_E_SHAPE
    # argmax: a 256-byte key/counter block per row; short or misaligned workspace; bad sizes
    assert lib.wsl_argmax_rows_workspace_bytes(8, 151936) == 8 * 256
    assert lib.wsl_argmax_rows_workspace_bytes(0, 10) == 0
    assert lib.wsl_argmax_rows_fwd(P2, 151936, 8, 151936, P2, P2, 8 * 256 - 1, None) == N.WSL_E_WORKSPACE
    assert lib.wsl_argmax_rows_fwd(P2, 151936, 8, 151936, P2, P2 + 16, 8 * 256, None) == N.WSL_E_WORKSPACE
    assert lib.wsl_argmax_rows_fwd(P2, 100, 8, 151936, P2, P2, 8 * 256, None) == N.WSL_E_SHAPE
    assert lib.wsl_argmax_rows_fwd(P2, 16, 0, 16, P2, None, 0, None) == N.WSL_OK


@needs_lib
@pytest.mark.parametrize("M,Nn,K,r,fuse,ok", [
    (8, 4096, 2048, 96, 1, 1),      # q|k|v of the bench model with the RMSNorm prologue
    (8, 12288, 2048, 32, 3, 1),     # gate|up with RMSNorm + SwiGLU
    (8, 2048, 6144, 16, 4, 1),      # down projection + residual
    (8, 256, 2048, 0, 1, 1),        # the head's first factor
    (8, 4096, 4096, 96, 1, 0),      # M * K / 8 chunks above what the prologue holds
    (8, 1000, 2048, 32, 3, 0),      # SwiGLU needs N % 16 == 0
    (8, 4096, 256, 16, 1, 0),       # short K: the fused kernels take 8 waves along K
    (8, 2048, 2048, 16, 6, 0),      # SwiGLU and residual exclude each other
    (65, 2048, 2048, 16, 4, 0),     # not decode-shaped
    (8, 2048, 2048, 12, 4, 0),      # r % 8 != 0
])
def test_fused_supported_answers_from_sizes(M, Nn, K, r, fuse, ok):
    assert N.lib().wsl_lora_linear_fused_supported(M, Nn, K, r, fuse) == ok
    assert N.last_error() == ""


def _fused(**kw):
    a = dict(x=P, ldx=2048, nw=P, eps=1e-6, w=P, ldw=2048, a=P, lda=2048, b=P, ldb=16, scale=2.0,
             res=None, ldr=0, y=P, ldy=4096, M=8, N=4096, K=2048, r=16, fuse=1, ws=P, ws_bytes=1 << 24)
    a.update(kw)
    return N.lib().wsl_lora_linear_fused_fwd(a["x"], a["ldx"], a["nw"], a["eps"], a["w"], a["ldw"], a["a"],
                                             a["lda"], a["b"], a["ldb"], a["scale"], a["res"], a["ldr"], a["y"],
                                             a["ldy"], a["M"], a["N"], a["K"], a["r"], a["fuse"], a["ws"],
                                             a["ws_bytes"], None)


@needs_lib
@pytest.mark.parametrize("kw,code", [
    (dict(fuse=0), N.WSL_E_INVALID_ARG),
    (dict(fuse=8), N.WSL_E_INVALID_ARG),
    (dict(fuse=6, N=2048, ldy=2048, res=P, ldr=2048), N.WSL_E_INVALID_ARG),
    (dict(nw=None), N.WSL_E_INVALID_ARG),
    (dict(fuse=4), N.WSL_E_INVALID_ARG),                    # residual missing
    (dict(M=65), N.WSL_E_SHAPE),
    (dict(fuse=3, N=1000, ldy=500), N.WSL_E_SHAPE),         # SwiGLU with N % 16 != 0
    (dict(fuse=3, ldy=2047), N.WSL_E_SHAPE),                # y is [M, N / 2]
    (dict(fuse=4, res=P, ldr=4000), N.WSL_E_SHAPE),
    (dict(K=4096, ldx=4096, ldw=4096, lda=4096), N.WSL_E_SHAPE),  # prologue capacity
    (dict(ws_bytes=1024), N.WSL_E_WORKSPACE),
    (dict(ws=P + 16), N.WSL_E_ALIGN),
])
def test_fused_validation_codes(kw, code):
    assert _fused(**kw) == code
    assert N.last_error() != ""


@needs_lib
def test_fused_empty_batch_is_a_no_op():
    assert _fused(M=0, x=None, y=None, ws=None, ws_bytes=0) == N.WSL_OK


def _grouped(group_n=(64, 64), **kw):
    a = dict(x=P, ldx=64, w=P, ldw=64, w_dtype=0, w_scale=None, a=P, lda=64, b=P, ldb=8,
             scale=2.0, y=P, ldy=128, M=4, K=64, r=8, ws=P, ws_bytes=1 << 24, stream=None)
    a.update(kw)
    gn = N.group_array(group_n) if group_n is not None else None
    ng = kw.get("n_groups", len(group_n) if group_n is not None else 2)
    return N.lib().wsl_lora_linear_grouped_fwd(a["x"], a["ldx"], a["w"], a["ldw"], a["w_dtype"], a["w_scale"],
                                               a["a"], a["lda"], a["b"], a["ldb"], a["scale"], a["y"], a["ldy"],
                                               a["M"], a["K"], a["r"], ng, gn, a["ws"], a["ws_bytes"],
                                               a["stream"])


@needs_lib
@pytest.mark.parametrize("group_n,kw,code", [
    ((64, 64), dict(n_groups=0), N.WSL_E_SHAPE),
    ((64,) * 5, {}, N.WSL_E_SHAPE),                   # more than WSL_MAX_GROUPS
    ((64, 0), {}, N.WSL_E_SHAPE),                     # empty group
    (None, dict(n_groups=2), N.WSL_E_INVALID_ARG),    # group_n NULL
    ((64, 64), dict(ldy=127), N.WSL_E_SHAPE),         # ldy < sum of widths
    ((64, 64), dict(x=None), N.WSL_E_INVALID_ARG),
    ((64, 64), dict(a=None), N.WSL_E_INVALID_ARG),
    ((64, 64), dict(w_dtype=1), N.WSL_E_INVALID_ARG),  # fp8 without w_scale
    ((64, 64), dict(lda=63), N.WSL_E_SHAPE),
    ((64, 64), dict(x=P + 1), N.WSL_E_ALIGN),
    ((64, 64), dict(ws=None), N.WSL_E_WORKSPACE),
    ((64, 64), dict(ws_bytes=16), N.WSL_E_WORKSPACE),
])
def test_grouped_validation_codes(group_n, kw, code):
    assert _grouped(group_n, **kw) == code
    assert N.last_error() != ""


@needs_lib
def test_grouped_empty_batch_is_a_no_op():
    assert _grouped((64, 64), M=0, x=None, y=None, ws=None, ws_bytes=0) == N.WSL_OK


@needs_lib
def test_grouped_workspace_covers_pre_pass_and_per_group_calls():
    # rank 128 over 3 groups: one pre-pass over 384 ranks (T [M, 384] plus split partials)
    M, K, r, gn = 4096, 4096, 128, (2048, 1024, 1024)
    need = N.grouped_workspace_bytes(M, K, r, gn, N.WSL_DTYPE_BF16)
    assert need >= _header_defines()["WSL_COUNTER_BYTES"] + M * 3 * r * 2
    for n in gn:  # the per-group fallback reuses the same workspace
        assert need >= N.workspace_bytes(M, n, K, r, N.WSL_DTYPE_BF16)
    # decode-shaped M: per-group calls
    assert N.grouped_workspace_bytes(8, 2048, 64, gn, 0) >= N.workspace_bytes(8, 2048, 2048, 64, 0)


def _noalloc(**kw):
    a = dict(x=P, ldx=64, w=P, ldw=64, w_dtype=0, w_scale=None, a=P, lda=64, b=P, ldb=8,
             scale=2.0, y=P, ldy=64, M=4, N=64, K=64, r=8, stream=None)
    a.update(kw)
    return N.lib().wsl_lora_linear_fwd_noalloc(a["x"], a["ldx"], a["w"], a["ldw"], a["w_dtype"], a["w_scale"],
                                               a["a"], a["lda"], a["b"], a["ldb"], a["scale"], a["y"], a["ldy"],
                                               a["M"], a["N"], a["K"], a["r"], a["stream"])


@needs_lib
@pytest.mark.parametrize("kw,code", [
    (dict(x=None), N.WSL_E_INVALID_ARG),
    (dict(w=None, r=0), N.WSL_E_INVALID_ARG),
    (dict(ldx=63), N.WSL_E_SHAPE),
    (dict(w_dtype=5), N.WSL_E_DTYPE),
    (dict(y=P + 1), N.WSL_E_ALIGN),
    # prefill rank pre-pass whose T alone is 32 MB: twice that (the workspace halves) and the
    # counter prefix exceed the static scratch, refused before any device is touched
    (dict(M=65536, N=1024, K=64, r=256, ldx=64, ldw=64, lda=64, ldb=256, ldy=1024), N.WSL_E_WORKSPACE),
])
def test_noalloc_validation_codes(kw, code):
    assert _noalloc(**kw) == code
    assert N.last_error() != ""


@needs_lib
def test_noalloc_empty_batch_is_a_no_op():
    assert _noalloc(M=0, x=None, y=None) == N.WSL_OK


def test_noalloc_scratch_size_matches_header():
    assert N.WSL_NOALLOC_SCRATCH_BYTES == 64 * 1024 * 1024
    text = open(HEADER).read()
    assert "#define WSL_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)" in text


def _bwd_weights(**kw):
    a = dict(x=P, ldx=64, gy=P, ldg=128, a=P, lda=64, b=P, ldb=8, scale=2.0, M=4, N=128, K=64, r=8,
             dw=P, lddw=64, da=P, ldda=64, db=P, lddb=8, ws=None, ws_bytes=0, stream=None)
    a.update(kw)
    return N.lib().wsl_lora_linear_bwd_weights(a["x"], a["ldx"], a["gy"], a["ldg"], a["a"], a["lda"], a["b"],
                                               a["ldb"], a["scale"], a["M"], a["N"], a["K"], a["r"], a["dw"],
                                               a["lddw"], a["da"], a["ldda"], a["db"], a["lddb"], a["ws"],
                                               a["ws_bytes"], a["stream"])


@needs_lib
@pytest.mark.parametrize("kw,code", [
    (dict(x=None), N.WSL_E_INVALID_ARG),
    (dict(a=None), N.WSL_E_INVALID_ARG),
    (dict(r=0), N.WSL_E_INVALID_ARG),            # da, db asked for without a rank
    (dict(ldx=63), N.WSL_E_SHAPE),
    (dict(ldg=127), N.WSL_E_SHAPE),
    (dict(lddb=7), N.WSL_E_SHAPE),
    (dict(dw=P + 1), N.WSL_E_ALIGN),
    (dict(x=P + 1), N.WSL_E_ALIGN),              # x not aligned to its element size
    (dict(K=72, ldx=72, lda=72, lddw=72, ldda=72), N.WSL_E_WORKSPACE),  # K off the grid: taken
    (dict(x=P + 2), N.WSL_E_WORKSPACE),          # x not 16-byte aligned: taken (scalar kernels)
    (dict(), N.WSL_E_WORKSPACE),                 # no workspace
])
def test_bwd_weights_validation_codes(kw, code):
    """Every refusal happens on the host, before any device is touched."""
    assert _bwd_weights(**kw) == code
    assert N.last_error() != ""


@needs_lib
def test_bwd_weights_nothing_to_do_is_a_no_op():
    assert _bwd_weights(M=0, x=None, gy=None) == N.WSL_OK
    assert _bwd_weights(dw=None, da=None, db=None) == N.WSL_OK


@needs_lib
@pytest.mark.parametrize("K,r,x,ok", [(64, 8, P, 1), (72, 8, P, 0), (64, 12, P, 0), (64, 8, P + 8, 0), (64, 0, P, 1)])
def test_bwd_weights_supported_answers_from_layout(K, r, x, ok):
    L = N.lib()
    assert L.wsl_lora_linear_bwd_weights_supported(x, K, P, 128, P, K, P, max(r, 8), 256, 128, K, r) == ok
    assert N.last_error() == ""


@needs_lib
def test_bwd_weights_workspace_holds_dw_copies_and_partials():
    """The weight-gradient workspace holds, in each half beside the counter prefix, the bf16 dW
    copy and dW^T of the dW route and the fp32 split partials (4 splits of 1024 x 1024 at
    M = 8192), and nothing the size of x or gy (the operands are read where they lie)."""
    M, Nn, K, r = 8192, 1024, 1024, 32
    got = N.bwd_weights_workspace_bytes(M, Nn, K, r)
    assert got >= 65536 + 2 * (2 * Nn * K * 2 + 4 * Nn * K * 4)
    assert got < 65536 + 2 * (K + Nn) * M * 2
    assert N.bwd_weights_workspace_bytes(0, Nn, K, r) >= 65536


def _bwd_input(**kw):
    a = dict(gy=P, ldg=128, w=P, ldw=64, w_dtype=N.WSL_DTYPE_BF16, w_scale=None, a=P, lda=64, b=P, ldb=8, scale=2.0,
             dx=P, lddx=64, M=4, N=128, K=64, r=8, ws=None, ws_bytes=0, stream=None)
    a.update(kw)
    return N.lib().wsl_lora_linear_bwd_input(a["gy"], a["ldg"], a["w"], a["ldw"], a["w_dtype"], a["w_scale"], a["a"],
                                             a["lda"], a["b"], a["ldb"], a["scale"], a["dx"], a["lddx"], a["M"], a["N"],
                                             a["K"], a["r"], a["ws"], a["ws_bytes"], a["stream"])


@needs_lib
@pytest.mark.parametrize("kw,code", [
    (dict(gy=None), N.WSL_E_INVALID_ARG),
    (dict(w=None), N.WSL_E_INVALID_ARG),
    (dict(b=None), N.WSL_E_INVALID_ARG),
    (dict(ldg=127), N.WSL_E_SHAPE),
    (dict(ldw=63), N.WSL_E_SHAPE),
    (dict(lddx=63), N.WSL_E_SHAPE),
    (dict(ldb=7), N.WSL_E_SHAPE),
    (dict(dx=P + 1), N.WSL_E_ALIGN),
    (dict(N=72, ldg=72), N.WSL_E_SHAPE),         # the reduction off the 64 grid: not taken
    (dict(gy=P + 8), N.WSL_E_SHAPE),             # gy rows not 16-byte aligned: not taken
    (dict(r=12, ldb=12), N.WSL_E_SHAPE),         # rank off 8
    (dict(w_dtype=7), N.WSL_E_DTYPE),
    (dict(w_dtype=N.WSL_DTYPE_FP8_E4M3), N.WSL_E_INVALID_ARG),              # fp8 without its scales
    (dict(w_dtype=N.WSL_DTYPE_FP8_E4M3, w_scale=P + 2), N.WSL_E_ALIGN),
    (dict(w_dtype=N.WSL_DTYPE_FP8_E4M3, w_scale=P, K=56, ldw=64, lda=64, lddx=64), N.WSL_E_SHAPE),  # K % 16
    (dict(w_dtype=N.WSL_DTYPE_FP8_E4M3, w_scale=P), N.WSL_E_WORKSPACE),     # fp8 taken
    (dict(), N.WSL_E_WORKSPACE),                 # no workspace
])
def test_bwd_input_validation_codes(kw, code):
    """Every refusal happens on the host, before any device is touched."""
    assert _bwd_input(**kw) == code
    assert N.last_error() != ""


@needs_lib
def test_bwd_input_empty_batch_and_queries():
    L = N.lib()
    assert _bwd_input(M=0, gy=None, dx=None) == N.WSL_OK
    bf = N.WSL_DTYPE_BF16
    assert L.wsl_lora_linear_bwd_input_supported(P, 128, P, 64, bf, None, P, 64, P, 8, P, 64, 4, 128, 64, 8) == 1
    assert L.wsl_lora_linear_bwd_input_supported(P, 128, P, 64, bf, None, None, 0, None, 0, P, 64, 4, 128, 64, 0) == 1
    assert L.wsl_lora_linear_bwd_input_supported(P, 100, P, 64, bf, None, P, 64, P, 8, P, 64, 4, 100, 64, 8) == 0
    assert L.wsl_lora_linear_bwd_input_supported(P, 128, P, 64, bf, None, P, 64, P, 8, P, 64, 4, 128, 60, 8) == 0
    f8 = N.WSL_DTYPE_FP8_E4M3
    assert L.wsl_lora_linear_bwd_input_supported(P, 128, P, 64, f8, P, P, 64, P, 8, P, 64, 4, 128, 64, 8) == 1
    assert L.wsl_lora_linear_bwd_input_supported(P, 128, P, 64, f8, None, P, 64, P, 8, P, 64, 4, 128, 64, 8) == 0
    assert L.wsl_lora_linear_bwd_input_supported(P, 128, P, 56, f8, P, P, 56, P, 8, P, 56, 4, 128, 56, 8) == 0
    assert N.last_error() == ""
    # the prefill scratch of the [M, K] outputs plus the transposed factors, and nothing the
    # size of W (read where it lies)
    M, Nn, K, r = 8192, 4096, 1024, 32
    got = N.bwd_input_workspace_bytes(M, Nn, K, r)
    assert got >= 65536 + 2 * (r * (Nn + K) * 2)
    assert got < 65536 + 2 * (Nn * K * 2)


@pytest.mark.parametrize("M,K", [(80, 256), (128, 640), (96, 2048), (65, 6144)])
def test_workspace_bytes_of_wide_decode_shapes(M, K):
    """65-128 tokens: the decode plan takes the shape or declines it (K not a multiple of its
    pass slice); either way the size queries give the bytes of a real path, not a wrapped
    subtraction."""
    for r in (0, 32):
        single = N.workspace_bytes(M, 3072, K, r, N.WSL_DTYPE_BF16)
        grouped = N.grouped_workspace_bytes(M, K, r, (1024, 512, 512), N.WSL_DTYPE_BF16)
        for b in (single, grouped):
            assert 0 < b < (1 << 32)


@pytest.mark.parametrize("M,Nn,K,r,splits", [
    (256, 2048, 2048, 64, 4),   # 32 tiles of 128 x 128, 32 K tiles: four splits of eight
    (256, 2048, 6144, 0, 8),    # 96 K tiles: eight splits fill 256 CUs
    (129, 1024, 1024, 16, 2),   # 16 K tiles: two splits of eight
    (160, 12288, 2048, 64, 0),  # 192 tiles: no split
])
def test_workspace_bytes_of_split_k_shapes(M, Nn, K, r, splits):
    """The in-launch split-K form's records (8 waves x 64 lanes x 16 words of 8 bytes per tile
    and split: the output partial, the LoRA term included) fit in the prefill half of the
    workspace the size query asks for, single and grouped."""
    tiles = ((M + 127) // 128) * ((Nn + 127) // 128)
    need = tiles * splits * 8 * 64 * 16 * 8
    half = lambda b: ((b - 65536) // 2) & ~255
    single = N.workspace_bytes(M, Nn, K, r, N.WSL_DTYPE_BF16)
    assert half(single) >= need
    if r:
        grouped = N.grouped_workspace_bytes(M, K, r, (Nn // 2, Nn // 4, Nn // 4), N.WSL_DTYPE_BF16)
        assert half(grouped) >= need


@needs_lib
def test_options_set_get_and_refuse():
    """Path overrides: every option round-trips, out-of-range values and unknown options are
    refused with WSL_E_INVALID_ARG and leave the value as it was."""
    d = _header_defines()
    for name, opt in N.OPTIONS.items():
        assert d["WSL_OPT_" + name.upper()] == opt
        assert N.get_option(name) == 0
    try:
        N.set_option("prefill_split", 4)
        assert N.get_option("prefill_split") == 4
        assert N.lib().wsl_set_option(N.OPTIONS["prefill_split"], 17) == N.WSL_E_INVALID_ARG
        assert N.lib().wsl_set_option(N.OPTIONS["prefill_strips"], 1) == N.WSL_E_INVALID_ARG
        assert N.lib().wsl_set_option(N.OPTIONS["decode_wide"], 2) == N.WSL_E_INVALID_ARG
        N.set_option("decode_wide", 1)
        assert N.get_option("decode_wide") == 1
        assert N.lib().wsl_set_option(N.OPTIONS["fp8_prefill"], -1) == N.WSL_E_INVALID_ARG
        assert N.lib().wsl_set_option(N.OPTIONS["fp8_prefill"], 3) == N.WSL_E_INVALID_ARG
        assert N.lib().wsl_set_option(N.OPTIONS["prefill_shared_t"], 3) == N.WSL_E_INVALID_ARG
        assert N.lib().wsl_set_option(N.OPTIONS["prefill_shared_t"], -2) == N.WSL_E_INVALID_ARG
        N.set_option("prefill_shared_t", 1)
        assert N.get_option("prefill_shared_t") == 1
        assert N.lib().wsl_set_option(99, 0) == N.WSL_E_INVALID_ARG
        assert N.lib().wsl_set_option(0, 0) == N.WSL_E_INVALID_ARG
        assert N.get_option("prefill_split") == 4
        with pytest.raises(ValueError):
            N.set_option("decode_passes", 2)
    finally:
        for name in N.OPTIONS:
            N.set_option(name, 0)


# Config 2 (Qwen3-0.6B, M = 8192, r = 32) and the 1.7B prefill launches: the tile each takes.
PLAN_CASES = [
    # M, K, r, groups, path, tile (m, n), rank blocks, strip tiles, workgroups
    (8192, 1024, 32, (2048, 1024, 1024), "prefill", (256, 256), 1, 2, 256),   # c2 q|k|v
    (8192, 2048, 32, (1024,), "prefill", (128, 256), 1, 1, 256),              # c2 o
    (8192, 1024, 32, (3072, 3072), "prefill", (256, 256), 1, 3, 256),         # c2 gate|up
    (8192, 3072, 32, (1024,), "prefill", (128, 256), 1, 1, 256),              # c2 down
    (8192, 2048, 32, (2048, 1024, 1024), "prefill", (256, 256), 1, 2, 256),   # 1.7b q|k|v
    (8192, 2048, 32, (2048,), "prefill", (256, 256), 1, 1, 256),              # 1.7b o
    (8192, 6144, 32, (2048,), "prefill", (256, 256), 1, 1, 256),              # 1.7b down
    (8192, 2048, 32, (6144, 6144), "prefill", (256, 256), 1, 6, 256),         # 1.7b gate|up
    (8192, 1024, 32, (3072,), "prefill", (256, 192), 1, 2, 256),              # c2 gate alone
]


@needs_lib
@pytest.mark.parametrize("M,K,r,groups,path,tile,rb,strips,wgs", PLAN_CASES)
def test_plan_of_benchmark_launches(M, K, r, groups, path, tile, rb, strips, wgs):
    p = N.plan(M, K, r, groups)
    assert p["path"] == path and (p["tile_m"], p["tile_n"]) == tile
    assert p["rank_blocks"] == rb and p["strip_tiles"] == strips and p["workgroups"] == wgs
    assert p["launches"] == 1 and p["k_splits"] == 1 and p["rank_prepass"] == 0


@needs_lib
def test_plan_shared_t_needs_a_device():
    """Shared T is taken for one wave of tiles on the current device, so the plan reads the
    device's CU count: on a host without a GPU it is never reported (the GPU tests assert
    where it is taken)."""
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible: tests/test_gpu_shared_t.py covers the plan there")
    assert N.plan(8192, 6144, 32, (2048,))["shared_t"] == 0
    assert N.plan(8192, 4096, 32, (1024,))["shared_t"] == 0


@needs_lib
def test_plan_follows_overrides():
    try:
        N.set_option("prefill_strips", -1)
        assert N.plan(8192, 1024, 32, (2048, 1024, 1024))["strip_tiles"] == 1
        N.set_option("prefill_strips", 0)
        assert N.plan(256, 2048, 64, (2048,))["path"] == "prefill_splitk"
        N.set_option("prefill_split", -1)
        assert N.plan(256, 2048, 64, (2048,))["path"] == "prefill"
        N.set_option("prefill_split", 2)
        p = N.plan(256, 2048, 64, (2048,))
        assert p["path"] == "prefill_splitk" and p["k_splits"] == 2
    finally:
        for name in N.OPTIONS:
            N.set_option(name, 0)


@needs_lib
def test_plan_split_form_needs_group_ends_on_its_tiles():
    """The in-launch split-K form runs 128 x 128 tiles that each compute one group's T. Group
    ends on multiples of 192 but not 128 must not reach it as one launch: the groups then run
    one by one (each may take the form alone); ends on multiples of 128 keep one launch."""
    p = N.plan(256, 4096, 16, (192, 192, 192))
    assert p["launches"] == 3
    assert N.plan(256, 4096, 16, (192,))["path"] == "prefill_splitk"
    p = N.plan(256, 4096, 16, (256, 128, 128))
    assert p["launches"] == 1 and p["path"] == "prefill_splitk"


@needs_lib
def test_plan_paths_by_size():
    assert N.plan(0, 1024, 16, (1024,))["path"] == "none"
    assert N.plan(8, 2048, 64, (2048, 1024, 1024))["path"] == "decode"
    assert N.plan(100, 1000, 16, (512,))["path"] == "generic"  # K off the 64 grid
    p = N.plan(4096, 4096, 128, (12288,), N.WSL_DTYPE_FP8_E4M3)  # 768 tiles of 256 x 256
    assert p["path"] == "prefill_fp8" and p["rank_prepass"] == 1
    # one wave of 256 x 256 tiles or less: W decoded onto the bf16 matrix cores, unless forced
    assert N.plan(4096, 4096, 128, (4096,), N.WSL_DTYPE_FP8_E4M3)["path"] == "prefill"
    assert N.plan(4096, 4096, 128, (1024,), N.WSL_DTYPE_FP8_E4M3)["path"] == "prefill"
    assert N.plan(4096, 4096, 128, (1024,), N.WSL_DTYPE_FP8_E4M3_ACT8)["path"] == "prefill_fp8"
    assert N.plan(4096, 4096, 128, (4096, 1024, 1024), N.WSL_DTYPE_FP8_E4M3)["path"] == "prefill_fp8"
    try:
        N.set_option("fp8_prefill", 2)
        assert N.plan(4096, 4096, 128, (1024,), N.WSL_DTYPE_FP8_E4M3)["path"] == "prefill_fp8"
        N.set_option("fp8_prefill", 1)
        assert N.plan(4096, 4096, 128, (12288,), N.WSL_DTYPE_FP8_E4M3)["path"] == "prefill"
    finally:
        N.set_option("fp8_prefill", 0)
    p = N.plan(4096, 4096, 128, (4096,))
    assert p["path"] == "prefill" and p["rank_prepass"] == 1 and p["rank_blocks"] == 0


@needs_lib
@pytest.mark.parametrize("M,K,r,groups,prepass,tile", [
    (8192, 2048, 64, (6144, 6144), 1, (256, 256)),   # 1.7B gate|up: T from the pre-pass frees 256 x 256
    (1024, 2048, 64, (6144, 6144), 1, (256, 192)),
    (512, 2048, 48, (6144, 6144), 1, (128, 256)),
    (256, 2048, 64, (6144, 6144), 0, (128, 128)),    # 128 x 128 either way: T in the loop
    (1024, 2048, 64, (2048, 1024, 1024), 0, (128, 128)),
    (8192, 2048, 32, (6144, 6144), 0, (256, 256)),   # one rank block: always in the loop
])
def test_plan_rank_33_to_64_takes_the_prepass_for_wider_tiles(M, K, r, groups, prepass, tile):
    """Ranks 33-64 take T from the rank pre-pass wherever that lets the launch use a tile
    wider than 128 x 128 (two in-loop rank blocks fit only 128 x 256 and 128 x 128)."""
    p = N.plan(M, K, r, groups)
    assert p["path"] == "prefill" and p["rank_prepass"] == prepass and (p["tile_m"], p["tile_n"]) == tile
    assert p["rank_blocks"] == (0 if prepass else (1 if r <= 32 else 2))
    if prepass:  # the size query covers the pre-pass's T and split partials
        assert N.grouped_workspace_bytes(M, K, r, groups, N.WSL_DTYPE_BF16) >= 65536 + 2 * M * r * len(groups) * 2
