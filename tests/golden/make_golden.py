"""Writes the small golden fixtures under tests/golden/ with plain Python loops.

The reference (muchanem/weightshared_torchtitan) ships no golden vectors for the LoRA
path, so these are computed from the definitions the reference's code spells out,
element by element, in Python floats (IEEE double), independently of numpy's matmul:

  lora_small.npz      y = x.W^T + s (x.A^T).B^T        model.py:189-192, 392-398
  broadcast_add.npz   out[h*D+d] = base[(h//(H/g))*D+d] + delta[h*D+d]   model.py:111-145
  fp8_table.npz       all 256 e4m3fn codes decoded from their bit fields
  fp8_quant.npz       per-channel e4m3fn quantisation by exhaustive nearest search
  embedding_small.npz out[t] = E[ids[t]].P^T, invalid id -> zero row

Inputs are drawn from random.Random(seed) and rounded to bf16 (ties to even) in pure
Python so the fixtures are exact on the bf16 grid. Run from the repo root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import random
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16(v: float) -> float:
    u = struct.unpack("<I", struct.pack("<f", v))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def randn_bf16(rng: random.Random, shape, std=1.0):
    n = 1
    for s in shape:
        n *= s
    flat = [bf16(rng.gauss(0.0, std)) for _ in range(n)]
    return flat, shape


def to_np(flat, shape):
    return np.array(flat, dtype=np.float64).reshape(shape)


def lora_loops(x, W, A, B, M, N, K, r, s):
    """y[m][n] = sum_k x[m][k] W[n][k] + s * sum_j (sum_k x[m][k] A[j][k]) B[n][j]."""
    y = []
    for m in range(M):
        t = []
        for j in range(r):
            acc = 0.0
            for k in range(K):
                acc += x[m * K + k] * A[j * K + k]
            t.append(acc)
        for n in range(N):
            base = 0.0
            if W is not None:
                for k in range(K):
                    base += x[m * K + k] * W[n * K + k]
            d = 0.0
            for j in range(r):
                d += t[j] * B[n * r + j]
            y.append(base + s * d)
    return y


def make_lora(rng):
    cases = {}
    specs = [
        # name, M, N, K, r, s, has_w
        ("c0", 5, 7, 16, 3, 2.0, True),
        ("c1", 4, 9, 24, 8, 2.0, True),
        ("c2", 3, 6, 10, 0, 2.0, True),     # plain linear (r = 0)
        ("c3", 6, 5, 12, 4, 2.0, False),    # delta only (LoRAModule.forward)
        ("c4", 2, 8, 32, 16, 1.0, True),    # scale 1 (config-5 convention)
        ("c5", 1, 11, 40, 4, 2.0, True),    # M = 1 (GEMV)
    ]
    for name, M, N, K, r, s, has_w in specs:
        x, _ = randn_bf16(rng, (M, K))
        W = randn_bf16(rng, (N, K), 0.2)[0] if has_w else None
        A, _ = randn_bf16(rng, (r, K), 0.2)
        B, _ = randn_bf16(rng, (N, r), 0.2)
        y = lora_loops(x, W, A, B, M, N, K, r, s)
        cases[f"{name}_x"] = to_np(x, (M, K))
        cases[f"{name}_W"] = to_np(W, (N, K)) if has_w else np.zeros((0, K))
        cases[f"{name}_A"] = to_np(A, (r, K))
        cases[f"{name}_B"] = to_np(B, (N, r))
        cases[f"{name}_s"] = np.array(s)
        cases[f"{name}_y"] = to_np(y, (M, N))
    cases["names"] = np.array([sp[0] for sp in specs])
    np.savez(os.path.join(HERE, "lora_small.npz"), **cases)


def make_broadcast_add(rng):
    cases = {}
    # (batch, H heads, D, g)
    specs = [("b0", 2, 4, 3, 2), ("b1", 3, 6, 2, 3), ("b2", 1, 4, 5, 4), ("b3", 2, 8, 2, 1)]
    for name, S, H, D, g in specs:
        base = [[rng.uniform(-1, 1) for _ in range(g * D)] for _ in range(S)]
        delta = [[rng.uniform(-1, 1) for _ in range(H * D)] for _ in range(S)]
        hpg = H // g
        out = [[base[s][(h // hpg) * D + d] + delta[s][h * D + d] for h in range(H) for d in range(D)]
               for s in range(S)]
        cases[f"{name}_base"] = np.array(base)
        cases[f"{name}_delta"] = np.array(delta)
        cases[f"{name}_g"] = np.array(g)
        cases[f"{name}_out"] = np.array(out)
    cases["names"] = np.array([sp[0] for sp in specs])
    np.savez(os.path.join(HERE, "broadcast_add.npz"), **cases)


def fp8_decode_bits(c: int) -> float:
    sign = -1.0 if c & 0x80 else 1.0
    e = (c >> 3) & 0xF
    m = c & 7
    if e == 0xF and m == 7:
        return float("nan")
    if e == 0:
        return sign * (m / 8.0) * 2.0 ** -6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def make_fp8(rng):
    table = np.array([fp8_decode_bits(c) for c in range(256)])
    np.savez(os.path.join(HERE, "fp8_table.npz"), values=table)
    # per-channel quantisation of a small W by exhaustive nearest search (ties -> even code)
    N, K = 6, 20
    W = [[rng.gauss(0.0, 0.02) for _ in range(K)] for _ in range(N)]
    W[2] = [0.0] * K  # all-zero row -> scale 1
    finite = [(c, fp8_decode_bits(c)) for c in range(0x7F)]
    scales, codes = [], []
    for n in range(N):
        amax = max(abs(v) for v in W[n])
        s = struct.unpack("<f", struct.pack("<f", amax / 448.0 if amax > 0 else 1.0))[0]
        scales.append(s)
        row = []
        for v in W[n]:
            a = min(abs(v / s), 448.0)
            best = None
            for c, val in finite:
                dist = abs(a - val)
                if best is None or dist < best[1] or (dist == best[1] and c % 2 == 0):
                    best = (c, dist)
            code = best[0] | (0x80 if v < 0 else 0)  # sign kept, as IEEE -0.0
            row.append(code)
        codes.append(row)
    np.savez(os.path.join(HERE, "fp8_quant.npz"), W=np.array(W), scales=np.array(scales, dtype=np.float32),
             codes=np.array(codes, dtype=np.uint8))


def make_embedding(rng):
    V, k, H = 11, 8, 6
    E, _ = randn_bf16(rng, (V, k))
    P, _ = randn_bf16(rng, (H, k), 0.3)
    ids = [3, 0, 10, -1, 7, 11, 3]  # -1 and 11 are out of range -> zero rows
    out = []
    for t in ids:
        for h in range(H):
            acc = 0.0
            if 0 <= t < V:
                for j in range(k):
                    acc += E[t * k + j] * P[h * k + j]
            out.append(acc)
    np.savez(os.path.join(HERE, "embedding_small.npz"), E=to_np(E, (V, k)), P=to_np(P, (H, k)),
             ids=np.array(ids, dtype=np.int64), out=to_np(out, (len(ids), H)))


if __name__ == "__main__":
    rng = random.Random(20261201)
    make_lora(rng)
    make_broadcast_add(rng)
    make_fp8(rng)
    make_embedding(rng)
    print("wrote fixtures to", HERE)
