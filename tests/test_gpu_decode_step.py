"""GPU parity of the decode-step kernels (include/wsl_decode.h) against plain PyTorch fp32
references of the same ops, at the benchmark model's shapes and at small/edge shapes.

Bar: max|y - y_ref| / max|y_ref| <= 1e-2 (bf16 output, fp32 arithmetic); bit-exact where
the op is exact (the bf16 residual sum, cache positions the step must not touch)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-2


def rel(x, ref):
    return ((x.float() - ref.float()).abs().max() / ref.float().abs().max()).item()


def _say(msg):
    print(msg, flush=True)


def rms_ref(h, w, eps):
    hf = h.float()
    return hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps) * w.float()


@pytest.mark.parametrize("rows,dim", [(8, 1024), (1, 2048), (3, 4096), (5, 8192), (16, 64)])
def test_rmsnorm_and_add_rmsnorm(gpu, rows, dim):
    from weightshared_torchtitan_amd import ops
    _say(f"[rmsnorm] rows={rows} dim={dim}")
    g = torch.Generator(device="cuda").manual_seed(rows * dim)
    x = torch.randn(rows, dim, device=gpu, generator=g).bfloat16()
    res = torch.randn(rows, dim, device=gpu, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(dim, device=gpu, generator=g)).bfloat16()
    out = ops.rmsnorm_op(x, w, 1e-6)
    assert rel(out, rms_ref(x, w, 1e-6)) <= TOL
    out2, h = ops.add_rmsnorm_op(x, res, w, 1e-6)
    h_ref = (x.float() + res.float()).bfloat16()
    assert torch.equal(h, h_ref)  # the residual sum is one bf16 rounding either way
    assert rel(out2, rms_ref(h_ref, w, 1e-6)) <= TOL


def rope_ref(x, rc_row, hd):
    cos, sin = rc_row[:hd], rc_row[hd:]
    rot = torch.cat((-x[..., hd // 2:], x[..., :hd // 2]), dim=-1)
    return x * cos + rot * sin


@pytest.mark.parametrize("b,nh,nkv,hd,L,pos", [(8, 16, 8, 128, 1024, 517), (2, 4, 2, 64, 32, 0),
                                             (3, 8, 8, 256, 16, 15)])
def test_qk_norm_rope_writes_q_and_cache(gpu, b, nh, nkv, hd, L, pos):
    from weightshared_torchtitan_amd import ops
    from weightshared_torchtitan_amd.qwen3_shared import _rope_cache
    _say(f"[qk_norm_rope] b={b} nh={nh} nkv={nkv} hd={hd} pos={pos}")
    g = torch.Generator(device="cuda").manual_seed(hd + pos)
    qkv = torch.randn(b, (nh + 2 * nkv) * hd, device=gpu, generator=g).bfloat16()
    qw = (1 + 0.1 * torch.randn(hd, device=gpu, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(hd, device=gpu, generator=g)).bfloat16()
    rope = _rope_cache(hd, L, 1e6).to(gpu)
    kc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
    vc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
    kc0, vc0 = kc.clone(), vc.clone()
    p = torch.full((), pos, dtype=torch.int64, device=gpu)
    q = ops.qk_norm_rope_op(qkv, qw, kw, 1e-6, rope, p, kc, vc, nh, nkv)
    heads = qkv.view(b, nh + 2 * nkv, hd).float()
    q_ref = rope_ref(rms_ref(heads[:, :nh], qw, 1e-6), rope[pos], hd)
    k_ref = rope_ref(rms_ref(heads[:, nh:nh + nkv], kw, 1e-6), rope[pos], hd)
    assert rel(q, q_ref) <= TOL
    assert rel(kc[:, :, pos], k_ref) <= TOL
    assert torch.equal(vc[:, :, pos], qkv.view(b, nh + 2 * nkv, hd)[:, nh + nkv:])
    others = torch.arange(L, device=gpu) != pos
    assert torch.equal(kc[:, :, others], kc0[:, :, others])
    assert torch.equal(vc[:, :, others], vc0[:, :, others])


def attn_ref(q, kc, vc, pos, scale):
    b, nh, hd = q.shape
    nkv = kc.shape[1]
    rep = nh // nkv
    k = kc[:, :, :pos + 1].float().repeat_interleave(rep, dim=1)   # [b, nh, t, hd]
    v = vc[:, :, :pos + 1].float().repeat_interleave(rep, dim=1)
    s = torch.einsum("bhd,bhtd->bht", q.float(), k) * scale
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bht,bhtd->bhd", p, v).reshape(b, nh * hd)


@pytest.mark.parametrize("b,nh,nkv,hd,L,pos", [(8, 16, 8, 128, 1024, 767), (8, 16, 8, 128, 1024, 0),
                                             (2, 4, 2, 64, 64, 37), (1, 8, 1, 128, 300, 299),
                                             (3, 4, 4, 64, 50, 31)])
def test_decode_attention(gpu, b, nh, nkv, hd, L, pos):
    from weightshared_torchtitan_amd import ops
    _say(f"[decode_attention] b={b} nh={nh} nkv={nkv} hd={hd} L={L} pos={pos}")
    g = torch.Generator(device="cuda").manual_seed(L + pos)
    q = torch.randn(b, nh, hd, device=gpu, generator=g).bfloat16()
    kc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
    vc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
    # positions past `pos` must not matter: fill them with huge values
    if pos + 1 < L:
        kc[:, :, pos + 1:] = 1e4
        vc[:, :, pos + 1:] = -1e4
    p = torch.full((), pos, dtype=torch.int64, device=gpu)
    out = ops.decode_attention_op(q, kc, vc, p, hd ** -0.5)
    ref = attn_ref(q, kc, vc, pos, hd ** -0.5)
    assert rel(out, ref) <= TOL


@pytest.mark.parametrize("rows,ffn", [(8, 3072), (1, 6144), (5, 64)])
def test_swiglu(gpu, rows, ffn):
    from weightshared_torchtitan_amd import ops
    _say(f"[swiglu] rows={rows} ffn={ffn}")
    g = torch.Generator(device="cuda").manual_seed(ffn)
    gu = torch.randn(rows, 2 * ffn, device=gpu, generator=g).bfloat16()
    out = ops.swiglu_op(gu)
    gf, uf = gu[:, :ffn].float(), gu[:, ffn:].float()
    assert rel(out, torch.nn.functional.silu(gf) * uf) <= TOL


def test_grouped_projection_equals_separate_calls(gpu):
    """[W_q; W_k; W_v] with the block-diagonal B is the three LoRA linears."""
    import weightshared_torchtitan_amd as wsl
    _say("[grouped qkv] M=8 K=1024 r=32")
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(8, 1024, device=gpu, generator=g).bfloat16()
    Ws = [(torch.randn(n, 1024, device=gpu, generator=g) * 0.02).bfloat16() for n in (2048, 1024, 1024)]
    As = [(torch.randn(32, 1024, device=gpu, generator=g) * 0.02).bfloat16() for _ in range(3)]
    Bs = [(torch.randn(n, 32, device=gpu, generator=g) * 0.02).bfloat16() for n in (2048, 1024, 1024)]
    sep = torch.cat([wsl.lora_linear(x, W, A, B, 2.0) for W, A, B in zip(Ws, As, Bs)], -1)
    Bbd = torch.zeros(4096, 96, device=gpu, dtype=torch.bfloat16)
    Bbd[:2048, :32], Bbd[2048:3072, 32:64], Bbd[3072:, 64:] = Bs
    grp = wsl.lora_linear(x, torch.cat(Ws), torch.cat(As), Bbd, 2.0)
    assert rel(grp, sep) <= 1e-2


@pytest.mark.parametrize("rows,n", [(8, 151936), (3, 1000), (2, 13), (16, 151936), (3, 4097), (5, 40000)])
def test_argmax_rows_matches_torch(gpu, rows, n):
    from weightshared_torchtitan_amd import ops
    _say(f"[argmax] rows={rows} n={n}")
    g = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn(rows, n, device=gpu, generator=g).bfloat16()
    x[0, n // 3] = 50.0          # unique maximum
    if rows > 1:
        x[1, 7 % n] = 60.0       # tie: the first index wins
        x[1, n - 1] = 60.0
    if rows > 2:
        x[2, n // 2] = float("nan")
    got = ops.argmax_rows_op(x)
    assert torch.equal(got, torch.argmax(x.float(), dim=-1))
    again = ops.argmax_rows_op(x)  # the split path's keys and counters were reset
    assert torch.equal(again, got)


def test_argmax_rows_edge_cases_and_paths(gpu):
    """Signed zeros tie (the first wins), several NaNs (the first wins), an all -inf row, and
    the one-workgroup-per-row path (no workspace) against the split path."""
    import ctypes
    from weightshared_torchtitan_amd import _native, ops
    n = 151936
    x = torch.full((4, n), -1.0, device=gpu, dtype=torch.bfloat16)
    x[0, 70000] = -0.0
    x[0, 90000] = 0.0
    x[1, 100] = float("nan")
    x[1, 50] = float("nan")
    x[1, 7] = float("inf")
    x[2, :] = float("-inf")
    x[3, 151935] = 3.0
    want = torch.argmax(x.float(), dim=-1)
    assert torch.equal(ops.argmax_rows_op(x), want)
    out = torch.empty(4, dtype=torch.int64, device=gpu)
    rc = _native.lib().wsl_argmax_rows_fwd(x.data_ptr(), x.stride(0), 4, n, out.data_ptr(), None, 0,
                                           torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == 0
    assert torch.equal(out, want)


@pytest.mark.parametrize("b,nh,nkv,hd,L,pos", [(8, 16, 8, 128, 1024, 767), (8, 16, 8, 128, 1024, 64),
                                             (2, 4, 2, 64, 64, 0), (3, 8, 2, 128, 200, 130),
                                             (2, 4, 4, 64, 80, 63), (2, 8, 2, 128, 4096, 3000)])
def test_decode_attention_step_equals_unfused(gpu, b, nh, nkv, hd, L, pos):
    """The fused step (norm + RoPE + cache write + split attention, merged by the last chunk
    to arrive) against the fp32 reference, twice in a row (arrival counters reset), and its
    cache writes equal to the unfused q/k-norm + RoPE kernel's."""
    from weightshared_torchtitan_amd import ops
    from weightshared_torchtitan_amd.qwen3_shared import _rope_cache
    _say(f"[attention step] b={b} nh={nh} nkv={nkv} hd={hd} L={L} pos={pos}")
    g = torch.Generator(device="cuda").manual_seed(3 * L + pos)
    qkv = torch.randn(b, (nh + 2 * nkv) * hd, device=gpu, generator=g).bfloat16()
    qw = (1 + 0.1 * torch.randn(hd, device=gpu, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(hd, device=gpu, generator=g)).bfloat16()
    rope = _rope_cache(hd, L, 1e6).to(gpu)
    kc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
    vc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
    kc2, vc2 = kc.clone(), vc.clone()
    p = torch.full((), pos, dtype=torch.int64, device=gpu)
    scale = hd ** -0.5
    q = ops.qk_norm_rope_op(qkv, qw, kw, 1e-6, rope, p, kc2, vc2, nh, nkv)
    ref = attn_ref(q, kc2, vc2, pos, scale)
    for _ in range(2):
        out = ops.decode_attention_step_op(qkv, qw, kw, 1e-6, rope, p, kc, vc, nh, nkv, scale)
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
        assert rel(out, ref) <= TOL
    ws = ops.workspace(gpu, torch.cuda.current_stream(gpu).cuda_stream, 0, kind="attention")
    assert int(ws[:65536].count_nonzero()) == 0, "arrival counters not restored to zero"



def test_decode_attention_step_workspace_shared_across_shapes(gpu):
    """One attention workspace serves calls of different shapes in turn: a call with few
    (sequence, kv head) pairs leaves records where a later call with more pairs might put
    counters, so the counters live in a fixed region of their own."""
    from weightshared_torchtitan_amd import ops
    from weightshared_torchtitan_amd.qwen3_shared import _rope_cache
    for (b, nh, nkv, hd, L, pos) in [(2, 4, 2, 64, 64, 0), (3, 8, 2, 128, 200, 130), (1, 4, 1, 64, 300, 299),
                                     (16, 16, 8, 64, 256, 200), (2, 4, 2, 64, 64, 10)]:
        _say(f"[attention step shared ws] b={b} nh={nh} nkv={nkv} hd={hd} L={L} pos={pos}")
        g = torch.Generator(device="cuda").manual_seed(7 * L + pos + b)
        qkv = torch.randn(b, (nh + 2 * nkv) * hd, device=gpu, generator=g).bfloat16()
        qw = (1 + 0.1 * torch.randn(hd, device=gpu, generator=g)).bfloat16()
        kw = (1 + 0.1 * torch.randn(hd, device=gpu, generator=g)).bfloat16()
        rope = _rope_cache(hd, L, 1e6).to(gpu)
        kc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
        vc = torch.randn(b, nkv, L, hd, device=gpu, generator=g).bfloat16()
        kc2, vc2 = kc.clone(), vc.clone()
        p = torch.full((), pos, dtype=torch.int64, device=gpu)
        scale = hd ** -0.5
        q = ops.qk_norm_rope_op(qkv, qw, kw, 1e-6, rope, p, kc2, vc2, nh, nkv)
        ref = attn_ref(q, kc2, vc2, pos, scale)
        out = ops.decode_attention_step_op(qkv, qw, kw, 1e-6, rope, p, kc, vc, nh, nkv, scale)
        assert rel(out, ref) <= TOL
    ws = ops.workspace(gpu, torch.cuda.current_stream(gpu).cuda_stream, 0, kind="attention")
    assert int(ws[:65536].count_nonzero()) == 0, "arrival counters not restored to zero"

def _interleave8(g, u):
    n = g.shape[0]
    return torch.stack((g.reshape(n // 8, 8, -1), u.reshape(n // 8, 8, -1)), 1).reshape(2 * n, -1).contiguous()


def _lora_ref(xb, W, A, B, s):
    """fp32 arithmetic on the bf16 input; T rounded to bf16 as the kernels publish it."""
    y = xb.float() @ W.float().t()
    if A is not None:
        t = (s * (xb.float() @ A.float().t())).bfloat16().float()
        y = y + t @ B.float().t()
    return y


@pytest.mark.parametrize("M,N,K,r,fuse", [
    (8, 4096, 2048, 96, 1),     # q|k|v of the benchmark model
    (1, 256, 1024, 16, 1),
    (16, 520, 1024, 32, 1),     # 16 * 1024 / 8: the prologue's full capacity
    (5, 1000, 3072, 24, 1),
    (2, 264, 1152, 8, 1),       # K / 8 = 144 chunks: 16-lane groups straddle wave boundaries
    (8, 256, 2048, 0, 1),       # the head's first factor (no adapter)
    (8, 12288, 2048, 32, 3),    # gate|up of the benchmark model
    (1, 512, 1024, 16, 3),
    (3, 2000, 1024, 24, 3),
    (8, 2048, 2048, 16, 4),     # o projection + residual
    (8, 2048, 6144, 16, 4),     # down projection + residual
    (5, 1000, 1024, 24, 4),     # N % 16 != 0: a partial last row block
    (64, 512, 1024, 8, 4),
    (4, 512, 1024, 16, 5),      # RMSNorm + residual
])
def test_fused_decode_linear(gpu, M, N, K, r, fuse):
    """The fused forms against the fp32 reference of the same composition, twice in a row
    (the launch and arrival counters carry over), and against the separate kernels."""
    from weightshared_torchtitan_amd import ops
    import weightshared_torchtitan_amd as wsl
    _say(f"[fused linear] M={M} N={N} K={K} r={r} fuse={fuse}")
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N + K + fuse)
    x = torch.randn(M, K, device=gpu, generator=g).bfloat16()
    nw = (1 + 0.1 * torch.randn(K, device=gpu, generator=g)).bfloat16() if fuse & 1 else None
    W = (torch.randn(N, K, device=gpu, generator=g) * K ** -0.5).bfloat16()
    A = (torch.randn(r, K, device=gpu, generator=g) * K ** -0.5).bfloat16() if r else None
    B = (torch.randn(N, r, device=gpu, generator=g) * 0.3).bfloat16() if r else None
    res = torch.randn(M, N, device=gpu, generator=g).bfloat16() if fuse & 4 else None
    s = 2.0
    xin = rms_ref(x, nw, 1e-6).bfloat16() if fuse & 1 else x
    y = _lora_ref(xin, W, A, B, s)
    if fuse & 2:
        # the same weights read as interleaved gate/up rows
        yv = y.view(M, N // 16, 2, 8)
        gate, up = yv[:, :, 0].reshape(M, N // 2), yv[:, :, 1].reshape(M, N // 2)
        ref = torch.nn.functional.silu(gate.bfloat16().float()) * up.bfloat16().float()
    else:
        ref = y
    if fuse & 4:
        ref = res.float() + y.bfloat16().float()
    for _ in range(2):
        out = ops.lora_linear_fused_op(x, nw, 1e-6, W, A, B, s, res, fuse)
        assert out.shape == ref.shape
        assert rel(out, ref) <= TOL
    # the separate kernels of the same step
    sep_in = ops.rmsnorm_op(x, nw, 1e-6) if fuse & 1 else x
    sep = wsl.lora_linear(sep_in, W, A, B, s) if r else wsl.lora_linear(sep_in, W)
    if fuse & 2:
        sv = sep.view(M, N // 16, 2, 8)
        gu = torch.cat([sv[:, :, 0].reshape(M, N // 2), sv[:, :, 1].reshape(M, N // 2)], 1)
        sep = ops.swiglu_op(gu)
    if fuse & 4:
        sep = (res.float() + sep.float()).bfloat16()
    assert rel(out, sep) <= TOL


def test_fused_swiglu_matches_separate_projections(gpu):
    """Interleaving gate/up rows (and B's rows, with A = [A1; A3] and B block-diagonal) is
    the two LoRA linears followed by SwiGLU."""
    from weightshared_torchtitan_amd import ops
    import weightshared_torchtitan_amd as wsl
    _say("[fused swiglu pack] M=8 F=3072 K=2048 r=16")
    g = torch.Generator(device="cuda").manual_seed(11)
    M, F, K, r = 8, 3072, 2048, 16
    x = torch.randn(M, K, device=gpu, generator=g).bfloat16()
    nw = (1 + 0.1 * torch.randn(K, device=gpu, generator=g)).bfloat16()
    W1, W3 = [(torch.randn(F, K, device=gpu, generator=g) * K ** -0.5).bfloat16() for _ in range(2)]
    A1, A3 = [(torch.randn(r, K, device=gpu, generator=g) * K ** -0.5).bfloat16() for _ in range(2)]
    B1, B3 = [(torch.randn(F, r, device=gpu, generator=g) * 0.3).bfloat16() for _ in range(2)]
    z = torch.zeros_like(B1)
    W = _interleave8(W1, W3)
    B = _interleave8(torch.cat([B1, z], 1), torch.cat([z, B3], 1))
    A = torch.cat([A1, A3], 0)
    out = ops.lora_linear_fused_op(x, nw, 1e-6, W, A, B, 2.0, None, 3)
    xn = ops.rmsnorm_op(x, nw, 1e-6)
    gate, up = wsl.lora_linear(xn, W1, A1, B1, 2.0), wsl.lora_linear(xn, W3, A3, B3, 2.0)
    ref = torch.nn.functional.silu(gate.float()) * up.float()
    assert rel(out, ref) <= TOL


def test_fused_unsupported_shape_raises(gpu):
    from weightshared_torchtitan_amd import ops
    x = torch.randn(8, 4096, device=gpu).bfloat16()
    W = torch.randn(256, 4096, device=gpu).bfloat16()
    nw = torch.ones(4096, device=gpu).bfloat16()
    assert not ops.lora_linear_fused_supported(8, 256, 4096, 0, 1)
    with pytest.raises(ValueError):
        ops.lora_linear_fused_op(x, nw, 1e-6, W, None, None, 0.0, None, 1)


# ------------------------------------------------------------------ tied head + greedy argmax
@pytest.mark.parametrize("M", [1, 8, 16, 17, 33, 64])
def test_tied_head_argmax_equals_argmax_of_logits(gpu, M):
    """The fused head (no logits written) gives torch.argmax of the bf16 logits the unfused
    head stores, bit for bit, at the config-4 head shape (vocab 151936, rank 256), over the
    plans M takes (one, two, three and four token blocks); twice in a row (the keys and the
    counter return to zero)."""
    from weightshared_torchtitan_amd import ops
    _say(f"[head argmax] M={M}")
    g = torch.Generator(device="cuda").manual_seed(100 + M)
    V, k = 151936, 256
    E = (torch.randn(V, k, device=gpu, generator=g) * 0.02).bfloat16()
    z = torch.randn(M, k, device=gpu, generator=g).bfloat16()
    assert ops.tied_head_argmax_supported(M, V, k)
    logits = ops.lora_linear(z, E, None, None, 0.0)  # the unfused head (same kernel sums)
    want = torch.argmax(logits, dim=-1)
    for _ in range(2):
        got = ops.tied_head_argmax_op(z, E)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    # against the fp32 logits: the chosen logit is within one bf16 rounding of the maximum
    ref = z.float() @ E.float().t()
    chosen = ref.gather(1, got[:, None])[:, 0]
    assert bool((chosen >= ref.max(-1).values - 2 ** -7 * ref.abs().max(-1).values).all())


@pytest.mark.parametrize("M,V", [(8, 40000), (40, 33000), (2, 32768)])
def test_tied_head_argmax_other_vocab_sizes(gpu, M, V):
    """Vocabularies whose workgroup count is not a multiple of the arrival groups (and whose
    last workgroup is partial): the same bit-for-bit bar, twice in a row."""
    from weightshared_torchtitan_amd import ops
    _say(f"[head argmax] M={M} V={V}")
    g = torch.Generator(device="cuda").manual_seed(V + M)
    k = 256
    E = (torch.randn(V, k, device=gpu, generator=g) * 0.02).bfloat16()
    z = torch.randn(M, k, device=gpu, generator=g).bfloat16()
    assert ops.tied_head_argmax_supported(M, V, k)
    want = torch.argmax(ops.lora_linear(z, E, None, None, 0.0), dim=-1)
    for _ in range(2):
        got = ops.tied_head_argmax_op(z, E)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_tied_head_argmax_ties_and_nan(gpu):
    """Ties give the first index and NaN counts as largest (the first NaN wins), as
    torch.argmax; placed in different workgroups' rows so the cross-workgroup merge decides."""
    from weightshared_torchtitan_amd import ops
    _say("[head argmax] ties and NaN")
    V, k, M = 151936, 256, 3
    g = torch.Generator(device="cuda").manual_seed(7)
    E = (torch.randn(V, k, device=gpu, generator=g) * 0.01).bfloat16()
    z = torch.ones(M, k, device=gpu).bfloat16()
    z[1] = -z[1]
    win = torch.full((k,), 0.5, device=gpu).bfloat16()
    for idx in (90001, 4242, 150000):      # row 0: equal maxima at three rows -> 4242
        E[idx] = win
    for idx in (120000, 777):              # row 1 (z negated): the same rows lose; its own tie
        E[idx] = -win
    nanrow = E[5].clone()
    nanrow[3] = float("nan")
    E[60000] = nanrow                      # every row of z meets a NaN at 60000 and at 140000
    E[140000] = nanrow
    got = ops.tied_head_argmax_op(z, E)
    torch.cuda.synchronize()
    want = torch.argmax(ops.lora_linear(z, E, None, None, 0.0), dim=-1)
    assert torch.equal(got, want)
    assert got.tolist() == [60000, 60000, 60000]
    E[60000] = E[6]
    E[140000] = E[7]
    got = ops.tied_head_argmax_op(z, E)
    torch.cuda.synchronize()
    assert got[0].item() == 4242 and got[1].item() == 777
    assert torch.equal(got, torch.argmax(ops.lora_linear(z, E, None, None, 0.0), dim=-1))


def test_tied_head_argmax_in_graph_replays(gpu):
    from weightshared_torchtitan_amd import ops
    _say("[head argmax] graph replays")
    V, k, M = 151936, 256, 8
    g = torch.Generator(device="cuda").manual_seed(9)
    E = (torch.randn(V, k, device=gpu, generator=g) * 0.02).bfloat16()
    z = torch.randn(M, k, device=gpu, generator=g).bfloat16()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.tied_head_argmax_op(z, E)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = ops.tied_head_argmax_op(z, E)
    for i in range(4):
        z.copy_(torch.randn(M, k, device=gpu, generator=g).bfloat16())
        graph.replay()
        torch.cuda.synchronize()
        want = torch.argmax(ops.lora_linear(z, E, None, None, 0.0), dim=-1)
        assert torch.equal(out, want), f"replay {i}"


@pytest.mark.parametrize("M,N,K,r", [(8, 1024, 2048, 32), (8, 1024, 3072, 32), (5, 1000, 1024, 24), (64, 512, 1024, 8)])
def test_fused_residual_in_place(gpu, M, N, K, r):
    """The residual epilogue with y aliasing the residual (the C ABI allows it): bit-equal
    to the out-of-place launch, since every workgroup reads the residual words it later
    overwrites before any of them is written."""
    import ctypes
    from weightshared_torchtitan_amd import ops, _native as N_
    _say(f"[fused residual in place] M={M} N={N} K={K} r={r}")
    g = torch.Generator(device="cuda").manual_seed(M + N + K + r)
    x = torch.randn(M, K, device=gpu, generator=g).bfloat16()
    W = (torch.randn(N, K, device=gpu, generator=g) * K ** -0.5).bfloat16()
    A = (torch.randn(r, K, device=gpu, generator=g) * K ** -0.5).bfloat16()
    B = (torch.randn(N, r, device=gpu, generator=g) * 0.3).bfloat16()
    res = torch.randn(M, N, device=gpu, generator=g).bfloat16()
    want = ops.lora_linear_fused_op(x, None, 1e-6, W, A, B, 2.0, res, N_.WSL_FUSE_RESIDUAL)
    h = res.clone()
    stream = ops._stream(h.device)
    ws = ops.workspace(h.device, stream, N_.workspace_bytes(M, N, K, r, N_.WSL_DTYPE_BF16))
    for _ in range(2):  # the second launch adds the delta to the first one's output
        h_prev = h.clone()
        rc = N_.lib().wsl_lora_linear_fused_fwd(
            x.data_ptr(), K, None, 1e-6, W.data_ptr(), K, A.data_ptr(), K, B.data_ptr(), r, 2.0,
            h.data_ptr(), N, h.data_ptr(), N, M, N, K, r, N_.WSL_FUSE_RESIDUAL, ws.data_ptr(), ws.numel(), stream)
        N_.check(rc, "wsl_lora_linear_fused_fwd")
        ref = ops.lora_linear_fused_op(x, None, 1e-6, W, A, B, 2.0, h_prev, N_.WSL_FUSE_RESIDUAL)
        torch.cuda.synchronize()
        assert torch.equal(h, ref)
    assert torch.equal(ops.lora_linear_fused_op(x, None, 1e-6, W, A, B, 2.0, res, N_.WSL_FUSE_RESIDUAL), want)
