"""Pins the CPU oracle: golden vectors from plain loops, known answers, invariants.

The reference ships no golden vectors for this path, so the fixtures under
tests/golden/ are computed element by element in Python (make_golden.py) from the
definitions in torchtitan/models/llama3/model/model.py:111-145,189-192,392-398.
"""
import os

import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ---------------------------------------------------------------- golden vectors
def test_lora_linear_matches_bruteforce_golden():
    g = _load("lora_small.npz")
    for name in g["names"]:
        x, W, A, B = g[f"{name}_x"], g[f"{name}_W"], g[f"{name}_A"], g[f"{name}_B"]
        s = float(g[f"{name}_s"])
        W = W if W.shape[0] > 0 else None
        y = O.lora_linear(x, W, A if A.shape[0] else None, B, s)
        np.testing.assert_allclose(y, g[f"{name}_y"], rtol=1e-12, atol=1e-12, err_msg=str(name))


def test_lora_delta_alone_matches_golden_delta_only_case():
    g = _load("lora_small.npz")
    y = O.lora_delta(g["c3_x"], g["c3_A"], g["c3_B"], float(g["c3_s"]))
    np.testing.assert_allclose(y, g["c3_y"], rtol=1e-12, atol=1e-12)


def test_broadcast_add_matches_index_formula_golden():
    g = _load("broadcast_add.npz")
    for name in g["names"]:
        out = O.broadcast_add(g[f"{name}_base"], g[f"{name}_delta"], dim=-1, g=int(g[f"{name}_g"]))
        np.testing.assert_allclose(out, g[f"{name}_out"], rtol=0, atol=0, err_msg=str(name))


def test_fp8_decode_matches_bitfield_table_and_known_answers():
    tab = _load("fp8_table.npz")["values"]
    dec = O.fp8_e4m3_decode(np.arange(256))
    np.testing.assert_array_equal(np.isnan(dec), np.isnan(tab))
    ok = ~np.isnan(tab)
    np.testing.assert_array_equal(dec[ok], tab[ok])
    assert dec[0x38] == 1.0 and dec[0x7E] == 448.0 and dec[0x08] == 2.0 ** -6 and dec[0x01] == 2.0 ** -9
    assert dec[0xB8] == -1.0 and np.isnan(dec[0x7F]) and np.isnan(dec[0xFF])


def test_fp8_decode_matches_torch_cast():
    codes = torch.arange(256, dtype=torch.uint8)
    t = codes.view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    dec = O.fp8_e4m3_decode(np.arange(256))
    ok = ~np.isnan(t)
    np.testing.assert_array_equal(np.isnan(dec), np.isnan(t))
    np.testing.assert_array_equal(dec[ok], t[ok])


def test_fp8_encode_roundtrip_and_torch_agreement():
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)])
    vals = O.fp8_e4m3_decode(finite)
    enc = O.fp8_e4m3_encode(vals)
    # -0.0 decodes to 0.0 then re-encodes as +0; every other code round-trips
    np.testing.assert_array_equal(enc[finite != 0x80], finite[finite != 0x80].astype(np.uint8))
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(20000) * 60).astype(np.float32)
    v = np.clip(v, -448, 448)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(O.fp8_e4m3_encode(v.astype(np.float64)), ref)


def test_fp8_quantize_matches_exhaustive_search_golden():
    g = _load("fp8_quant.npz")
    q, s = O.quantize_fp8_per_channel(g["W"])
    np.testing.assert_array_equal(s, g["scales"])
    np.testing.assert_array_equal(q, g["codes"])


def test_fp8_quantization_error_bound():
    rng = np.random.default_rng(1)
    W = rng.standard_normal((64, 256)) * 0.02
    q, s = O.quantize_fp8_per_channel(W)
    Wd = O.dequantize_fp8(q, s)
    scaled = np.abs(W / s[:, None].astype(np.float64))
    normal = scaled >= 2.0 ** -6
    # relative error of a 3-mantissa-bit grid is at most half an ulp = 2^-4
    assert np.all(np.abs(Wd - W)[normal] <= 2.0 ** -4 * np.abs(W)[normal] + 1e-30)


def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(2)
    v = rng.standard_normal(50000).astype(np.float32) * 3
    # exact ties: values whose low 16 bits are 0x8000
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32) * 1.0
    v = np.concatenate([v, ties[np.isfinite(ties)]])
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(v), ref)


def test_factorized_embedding_matches_golden():
    g = _load("embedding_small.npz")
    out = O.factorized_embedding(g["ids"], g["E"], g["P"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- invariants
@pytest.fixture(scope="module")
def case():
    rng = np.random.default_rng(3)
    M, N, K, r = 37, 29, 48, 6
    x = O.bf16_round(rng.standard_normal((M, K)))
    W = O.bf16_round(rng.standard_normal((N, K)) * 0.02)
    A = O.bf16_round(rng.standard_normal((r, K)) * 0.02)
    B = O.bf16_round(rng.standard_normal((N, r)) * 0.02)
    return x, W, A, B


def test_zero_b_or_zero_scale_reduces_to_matmul(case):
    x, W, A, B = case
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    np.testing.assert_allclose(O.lora_linear(x, W, A, np.zeros_like(B), 2.0), ref, rtol=0, atol=1e-15)
    np.testing.assert_allclose(O.lora_linear(x, W, A, B, 0.0), ref, rtol=0, atol=1e-15)
    np.testing.assert_allclose(O.lora_linear(x, W, None, None), ref, rtol=0, atol=0)


def test_linear_in_scale(case):
    x, W, A, B = case
    y1 = O.lora_linear(x, W, A, B, 1.0)
    y3 = O.lora_linear(x, W, A, B, 3.0)
    y0 = O.lora_linear(x, W, A, B, 0.0)
    np.testing.assert_allclose(y3 - y0, 3.0 * (y1 - y0), rtol=1e-10, atol=1e-12)


def test_rank_concatenation(case):
    x, W, A, B = case
    y = O.lora_linear(x, W, A, B, 2.0)
    y12 = O.lora_linear(x, W, A[:2], B[:, :2], 2.0) + O.lora_delta(x, A[2:], B[:, 2:], 2.0)
    np.testing.assert_allclose(y, y12, rtol=1e-12, atol=1e-14)


def test_rows_are_independent(case):
    x, W, A, B = case
    y = O.lora_linear(x, W, A, B, 2.0)
    for rows in (slice(0, 1), slice(5, 20), slice(36, 37)):
        np.testing.assert_allclose(O.lora_linear(x[rows], W, A, B, 2.0), y[rows], rtol=1e-12, atol=1e-14)


def test_transposed_operand_is_caught(case):
    # a plausible mistake (B used transposed via a square case) must change the answer
    x, W, A, B = case
    Bsq = O.bf16_round(np.random.default_rng(4).standard_normal((A.shape[0], A.shape[0])))
    y = O.lora_delta(x, A, Bsq, 2.0)
    y_bad = O.lora_delta(x, A, Bsq.T, 2.0)
    assert O.max_rel_err(y_bad, y) > 1e-2


def test_rounded_t_contract_close_to_exact(case):
    x, W, A, B = case
    y = O.lora_linear(x, W, A, B, 2.0)
    yt = O.lora_linear_rounded_t(x, W, A, B, 2.0)
    assert O.max_rel_err(yt, y) < 2e-3


def test_tied_logits_is_embedding_transpose():
    rng = np.random.default_rng(5)
    V, k, H = 13, 4, 6
    E = rng.standard_normal((V, k))
    P = rng.standard_normal((H, k))
    h = rng.standard_normal((3, H))
    logits = O.tied_logits(h, P, E)
    emb = O.factorized_embedding(np.arange(V), E, P)  # [V, H]
    np.testing.assert_allclose(logits, h @ emb.T, rtol=1e-12, atol=1e-12)


def test_embedding_identity_projection_is_lookup():
    rng = np.random.default_rng(6)
    E = rng.standard_normal((9, 5))
    ids = np.array([4, 4, 0, 8])
    np.testing.assert_array_equal(O.factorized_embedding(ids, E, np.eye(5)), E[ids])


def test_oracle_matches_reference_style_torch_cpu_path(case):
    # the reference's own CPU arithmetic: F.linear(x,W) + F.linear(F.linear(x,A),B)*s (fp32)
    from oracle.qwen3_ref import reference_lora_linear
    x, W, A, B = case
    t = lambda a: torch.from_numpy(np.asarray(a, np.float32))
    y_ref = reference_lora_linear(t(x), t(W), t(A), t(B), 2.0).numpy()
    assert O.max_rel_err(y_ref, O.lora_linear(x, W, A, B, 2.0)) < 1e-5


# ---------------------------------------------------------------- backward
def test_backward_matches_torch_autograd_float64(case):
    x, W, A, B = case
    gy = np.random.default_rng(7).standard_normal((x.shape[0], W.shape[0]))
    ws = np.random.default_rng(8).uniform(0.5, 2.0, W.shape[0])
    for w_scale in (None, ws):
        tx, tW, tA, tB = (torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, W, A, B))
        Wd = tW * torch.tensor(w_scale)[:, None] if w_scale is not None else tW
        y = tx @ Wd.T + 2.0 * (tx @ tA.T) @ tB.T
        y.backward(torch.tensor(gy))
        dx, dW, dA, dB = O.lora_linear_backward(x, W, A, B, 2.0, gy, w_scale=w_scale)
        np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(dA, tA.grad.numpy(), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(dB, tB.grad.numpy(), rtol=1e-12, atol=1e-12)
        gW = tW.grad.numpy() if w_scale is None else tW.grad.numpy() / w_scale[:, None]
        np.testing.assert_allclose(dW, gW, rtol=1e-10, atol=1e-12)


def test_backward_matches_central_differences():
    # brute force on a tiny case: L = <gy, y>, every input element perturbed in turn
    rng = np.random.default_rng(11)
    M, N, K, r = 3, 4, 5, 2
    x, W, A, B = (rng.standard_normal(s) for s in ((M, K), (N, K), (r, K), (N, r)))
    gy = rng.standard_normal((M, N))
    s, h = 1.7, 1e-6

    def loss(x_, W_, A_, B_):
        return float((O.lora_linear(x_, W_, A_, B_, s) * gy).sum())

    grads = O.lora_linear_backward(x, W, A, B, s, gy)
    args = [x, W, A, B]
    for which, g in enumerate(grads):
        num = np.zeros_like(args[which])
        for idx in np.ndindex(*args[which].shape):
            hi = [a.copy() for a in args]
            lo = [a.copy() for a in args]
            hi[which][idx] += h
            lo[which][idx] -= h
            num[idx] = (loss(*hi) - loss(*lo)) / (2 * h)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8)


def test_backward_dx_is_forward_with_transposed_weights(case):
    # dx = gy . W + s (gy . B) . A is the forward of the same op with W^T, B^T, A^T: the
    # identity the GPU backward uses to run dx on the forward kernel
    x, W, A, B = case
    gy = O.bf16_round(np.random.default_rng(9).standard_normal((x.shape[0], W.shape[0])))
    dx = O.lora_linear_backward(x, W, A, B, 2.0, gy)[0]
    np.testing.assert_allclose(O.lora_linear(gy, W.T, B.T, A.T, 2.0), dx, rtol=1e-12, atol=1e-13)
    # a dropped LoRA term or a flipped sign on it is caught
    assert O.max_rel_err(O.lora_linear(gy, W.T), dx) > 1e-3
    assert O.max_rel_err(O.lora_linear(gy, W.T, B.T, A.T, -2.0), dx) > 1e-3
