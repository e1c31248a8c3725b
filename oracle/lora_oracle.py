"""numpy restatement of the reference's LoRA-linear arithmetic (test infrastructure only).

Every function computes in float64 from inputs that are already on the storage grid
(bf16 values held in float32/float64 arrays), so it is the "fp32 reference" of the
north-star tolerance with headroom to spare.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = 448.0


# ----------------------------------------------------------------------------------------
# LoRA linear
# ----------------------------------------------------------------------------------------
def lora_delta(x, A, B, scale):
    """delta = w_b(w_a(x)) * (alpha / rank) = scale * (x . A^T) . B^T.

    Follows torchtitan/models/llama3/model/model.py:189-192 (LoRAModule.forward: two
    bias-free nn.Linear and a multiply by alpha/rank; alpha = 2*rank at :162).
    Pinned by: the brute-force golden vectors (tests/golden/lora_small.npz), the
    r-concatenation and linearity-in-scale invariants (tests/test_oracle.py).
    """
    x = np.asarray(x, dtype=np.float64)
    return (x @ np.asarray(A, np.float64).T) @ np.asarray(B, np.float64).T * float(scale)


def lora_linear(x, W, A=None, B=None, scale=2.0, w_scale=None):
    """y = base(x) + delta(x) with base(x) = x . W^T (* w_scale per output channel).

    Follows torchtitan/models/llama3/model/model.py:392-398: q_base = wq_base(x)
    (nn.Linear, bias=False, :257-273), wq_offset = LoRAModule(x) (:377), and
    broadcast_add(q_base, wq_offset, g) which is a plain add when base and delta have the
    same width (:111-145). W may be None (delta only) and A/B None (plain linear).
    Pinned by: golden vectors (brute-force triple loops), B = 0 and scale = 0 reduce to
    the textbook matmul, M-row independence (tests/test_oracle.py).
    """
    x = np.asarray(x, dtype=np.float64)
    y = None
    if W is not None:
        y = x @ np.asarray(W, np.float64).T
        if w_scale is not None:
            y = y * np.asarray(w_scale, np.float64)[None, :]
    if A is not None and A.shape[0] > 0:
        d = lora_delta(x, A, B, scale)
        y = d if y is None else y + d
    if y is None:
        raise ValueError("lora_linear needs W or (A, B)")
    return y


def lora_linear_rounded_t(x, W, A, B, scale, w_scale=None):
    """The kernel contract: T = bf16(scale * x . A^T) rounded once, y = base + T . B^T.

    Used to separate the one intended rounding of T from kernel error in tests.
    Pinned by: agrees with lora_linear up to the bf16 rounding of T (bounded in
    tests/test_oracle.py).
    """
    x = np.asarray(x, dtype=np.float64)
    y = x @ np.asarray(W, np.float64).T if W is not None else 0.0
    if W is not None and w_scale is not None:
        y = y * np.asarray(w_scale, np.float64)[None, :]
    if A is not None and A.shape[0] > 0:
        t = bf16_round(float(scale) * (x @ np.asarray(A, np.float64).T))
        y = y + t.astype(np.float64) @ np.asarray(B, np.float64).T
    return y


def max_rel_err(y, y_ref):
    """max|y - y_ref| / max|y_ref| (the north-star correctness metric)."""
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    denom = np.abs(y_ref).max()
    return float(np.abs(y - y_ref).max() / (denom if denom > 0 else 1.0))


# ----------------------------------------------------------------------------------------
# broadcast_add (head-sharing composition)
# ----------------------------------------------------------------------------------------
def broadcast_add(base, delta, dim=-1, g=1):
    """broadcast(base) + delta, base = g templates of width D shared by H/g heads each.

    Follows torchtitan/models/llama3/model/model.py:111-145 (reshape base to (g, D),
    insert a heads-per-group axis, expand, flatten to delta's shape, add).
    Pinned by: the explicit index formula out[h*D + d] = base[(h // (H/g))*D + d] +
    delta[h*D + d] evaluated element by element in tests/golden (broadcast_add.npz), and
    g*D == H*D reducing to a plain add.
    """
    base = np.asarray(base)
    delta = np.asarray(delta)
    if dim < 0:
        dim += base.ndim
    big, small = delta.shape[dim], base.shape[dim]
    assert big % small == 0, "delta and base feature dims incompatible"
    hpg = big // small
    d = small // g
    shp = list(base.shape)
    shp[dim:dim + 1] = [g, 1, d]
    b = base.reshape(shp)
    tile = [1] * b.ndim
    tile[dim + 1] = hpg
    b = np.tile(b, tile).reshape(delta.shape)
    return b + delta


# ----------------------------------------------------------------------------------------
# bf16 / fp8 encodings
# ----------------------------------------------------------------------------------------
def bf16_round(a):
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32.

    Pinned by: agrees bit for bit with torch's float32 -> bfloat16 cast on random and
    tie-case inputs (tests/test_oracle.py).
    """
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def fp8_e4m3_decode(codes):
    """OCP float8_e4m3fn code -> float64 (1 sign, 4 exponent bits with bias 7, 3 mantissa
    bits; exponent 0 is subnormal, S.1111.111 is NaN, there is no infinity).

    Pinned by: the all-256-codes table built by a pure-Python bit formula in
    tests/golden (fp8_table.npz), known answers (0x38 = 1.0, 0x7E = 448, 0x08 = 2^-6,
    0x01 = 2^-9), and torch's float8_e4m3fn -> float32 cast.
    """
    c = np.asarray(codes).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = (c & 0x7).astype(np.float64)
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    val = np.where((e == 0xF) & ((c & 7) == 7), np.nan, val)
    return sign * val


_FP8_POS = np.array([fp8_e4m3_decode(c) for c in range(0x7F)], dtype=np.float64)  # codes 0..126


def fp8_e4m3_encode(v):
    """float -> nearest float8_e4m3fn code (ties to the even code), saturating at 448.

    Pinned by: round-trips every finite code exactly, and agrees with torch's
    float32 -> float8_e4m3fn cast on random inputs (tests/test_oracle.py).
    """
    v = np.asarray(v, dtype=np.float64)
    a = np.minimum(np.abs(v), FP8_MAX)
    idx = np.searchsorted(_FP8_POS, a)  # first table value >= a
    idx = np.clip(idx, 1, len(_FP8_POS) - 1)
    lo, hi = _FP8_POS[idx - 1], _FP8_POS[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & ((idx % 2) == 0))
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(a == 0, 0, code)
    return (code | np.where(v < 0, 0x80, 0)).astype(np.uint8)


def quantize_fp8_per_channel(W):
    """s_n = max|W_n| / 448, Q = e4m3fn(W / s_n) (all-zero rows: s_n = 1).

    Restates the config-5 weight quantisation (per-output-channel, weight-only); the
    reference has no such quantiser (its fp8 path is torchao training fp8,
    torchtitan/components/quantization/float8.py:26-218).
    Pinned by: the brute-force quantisation fixture (tests/golden/fp8_quant.npz) and the
    bound |Q*s - W| <= 2^-4 |W| for normal values (tests/test_oracle.py).
    """
    W = np.asarray(W, dtype=np.float64)
    amax = np.abs(W).max(axis=1)
    s = np.where(amax > 0, amax / FP8_MAX, 1.0).astype(np.float32).astype(np.float64)
    q = fp8_e4m3_encode(W / s[:, None])
    return q, s.astype(np.float32)


def dequantize_fp8(q, s):
    return fp8_e4m3_decode(q) * np.asarray(s, np.float64)[:, None]


FP8_LO_SHIFT = 4  # the low activation term carries the residual times 2^4


def fp8_token_exponent(x):
    """Per-row power-of-two scale exponent of the fp8 activations: the smallest integer e
    with max|x[m]| * 2^-e <= 448 (0 for an all-zero row), clamped to [-126, 127].

    The build's own fp8-activation scheme (the reference's fp8 is torchao's dynamic
    training recipe, torchtitan/components/quantization/float8.py:26-218, absent here).
    With f = max|x[m]| = mf * 2^ef, mf in [1, 2): e = ef - 8 + (mf > 1.75), since
    448 = 1.75 * 2^8. Pinned by: brute-force search for the smallest such e on random and
    edge-case rows (tests/test_fp8_activation_cpu.py).
    """
    x = np.asarray(x, np.float64)
    amax = np.abs(x).max(axis=-1)
    m, ex = np.frexp(amax)          # amax = m * 2^ex, m in [0.5, 1)
    e = (ex - 1) - 8 + (2.0 * m > 1.75)
    e = np.where(amax > 0, e, 0)
    return np.clip(e, -126, 127).astype(np.int64)


def fp8_split_activations(x, terms=2):
    """Activations x [M, K] (bf16 values) as `terms` e4m3 codes per element and a per-row
    exponent e: x[m, k] ~= 2^e[m] * (dec(c[0, m, k]) + 2^-4 dec(c[1, m, k])).

    c[0] = e4m3(x * 2^-e) rounded to nearest even; c[1] = e4m3((x * 2^-e - dec(c[0])) * 2^4),
    the rounding residual one e4m3 step further down. Every step but the two roundings is
    exact (power-of-two scaling; the residual of a bf16 value against its e4m3 rounding is
    an fp32 value). With two terms a bf16 value is carried to within 2^-8 of itself, so the
    fp8 MFMA sees bf16-quality activations.
    Pinned by: a per-element pure-Python restatement on a tiny case, exact reconstruction
    of bf16 values, and the error bounds of tests/test_fp8_activation_cpu.py.
    """
    x = np.asarray(x, np.float64)
    e = fp8_token_exponent(x)
    xs = x * np.exp2(-e.astype(np.float64))[:, None]
    hi = fp8_e4m3_encode(xs)
    codes = [hi]
    if terms >= 2:
        res = (xs - fp8_e4m3_decode(hi)) * 2.0 ** FP8_LO_SHIFT
        codes.append(fp8_e4m3_encode(res))
    return np.stack(codes), e


def fp8_activations_value(codes, e):
    """The activations the fp8 MFMA path multiplies: 2^e * sum_t 2^(-4 t) dec(codes[t])."""
    v = sum(fp8_e4m3_decode(codes[t]) * 2.0 ** (-FP8_LO_SHIFT * t) for t in range(codes.shape[0]))
    return v * np.exp2(np.asarray(e, np.float64))[:, None]


# ----------------------------------------------------------------------------------------
# factorized embedding + tied output
# ----------------------------------------------------------------------------------------
def factorized_embedding(ids, E, P):
    """out[t] = E[ids[t]] . P^T; ids outside [0, V) give a zero row.

    The reference has a full-rank nn.Embedding(vocab, dim)
    (torchtitan/models/llama3/model/model.py:561); this is its rank-k factorisation
    (gather, then nn.Linear(k, dim) with weight P [dim, k]).
    Pinned by: golden vectors (tests/golden/embedding_small.npz) from explicit loops,
    and k == dim with P = I reducing to the plain embedding lookup.
    """
    ids = np.asarray(ids).reshape(-1)
    E = np.asarray(E, np.float64)
    valid = (ids >= 0) & (ids < E.shape[0])
    rows = np.where(valid[:, None], E[np.where(valid, ids, 0)], 0.0)
    return rows @ np.asarray(P, np.float64).T


def tied_logits(h, P, E):
    """logits = (h . P) . E^T — the output head tied to the factorized embedding.

    Pinned by: equals factorized_embedding's transpose identity
    <tied_logits(h)[t, v]> = <h[t], factorized_embedding([v])> (tests/test_oracle.py).
    """
    return (np.asarray(h, np.float64) @ np.asarray(P, np.float64)) @ np.asarray(E, np.float64).T


# ----------------------------------------------------------------------------------------
# Backward of the LoRA linear
# ----------------------------------------------------------------------------------------
def lora_linear_backward(x, W, A, B, scale, gy, w_scale=None):
    """Gradients of y = x . (W * w_scale[:, None])^T + scale * (x . A^T) . B^T w.r.t. x, W,
    A and B, given dL/dy = gy. Returns (dx, dW, dA, dB); dW is None when W is None and
    dA, dB are None without a LoRA term. For an fp8 W, dW is the gradient w.r.t. the
    dequantised weight W * w_scale[:, None].

    The reference has no backward of its own: torch autograd differentiates
    LoRAModule.forward (torchtitan/models/llama3/model/model.py:189-192, two bias-free
    nn.Linear and a multiply) and the base nn.Linear (:257-273) composed by broadcast_add
    with g = 1 (:392-398); the trainer runs it at torchtitan/train.py:456. With
    T = x . A^T and U = gy . B:
        dx = gy . W + scale * U . A,   dW = gy^T . x,
        dA = scale * U^T . x,          dB = scale * gy^T . T.
    Pinned by: torch.autograd of the same expression in float64, and central finite
    differences of a scalar loss on tiny shapes (tests/test_oracle.py).
    """
    x = np.asarray(x, np.float64)
    gy = np.asarray(gy, np.float64)
    dx = np.zeros_like(x)
    dW = dA = dB = None
    if W is not None:
        Wd = np.asarray(W, np.float64)
        if w_scale is not None:
            Wd = Wd * np.asarray(w_scale, np.float64)[:, None]
        dx = dx + gy @ Wd
        dW = gy.T @ x
    if A is not None and A.shape[0] > 0:
        A = np.asarray(A, np.float64)
        B = np.asarray(B, np.float64)
        U = gy @ B
        T = x @ A.T
        dx = dx + float(scale) * (U @ A)
        dA = float(scale) * (U.T @ x)
        dB = float(scale) * (gy.T @ T)
    return dx, dW, dA, dB
