"""Write the small golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no test vectors for this path, so these fixtures are the
oracle's outputs on seeded inputs (bf16 tensors stored as raw uint16 bits).
They lock the oracle against regressions (CPU tests) and give the GPU tests
fixed cases with planted ties, a ragged vocabulary tail and an all -inf row.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def bf16(rng, shape, std=1.0):
    return oracle.bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def bits(x):
    return oracle.f32_to_bf16_bits(x).reshape(np.shape(x))


def argmax_case(seed, M, d, r, V, act, base_bf16, with_prior, plant):
    rng = np.random.default_rng(seed)
    h = bf16(rng, (M, d))
    A = bf16(rng, (r, d), 0.02)
    B = bf16(rng, (V, r), 0.02)
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    prior = np.log(rng.dirichlet(np.ones(V) * 0.5) + 1e-12).astype(np.float32)
    if base_bf16:
        base, prior = oracle.bf16_round(base), oracle.bf16_round(prior)
    alpha = rng.uniform(0, 0.6, M).astype(np.float32)
    beta = rng.uniform(0, 0.6, M).astype(np.float32)
    beta[M // 2] = 0.0
    if plant:
        B[[3, V - 1, 17, V - 17, 500 % V]] = 0.0
        prior[[3, V - 1, 17, V - 17, 500 % V]] = 0.0
        base[0, V - 1] = 50.0                       # maximum in the ragged tail
        base[1, 17] = base[1, V - 17] = 50.0        # tie far apart -> lower index
        base[2, 3] = base[2, 500 % V] = 50.0        # tie -> lower index
        base[M - 1, :] = -np.inf                    # all -inf row -> id 0
        alpha[M - 1] = 0.0
    rank = oracle.rank_proj(h, A, None, act)
    ids, score, second = oracle.fused_argmax(rank, B, base, prior if with_prior else None, alpha, beta)
    return dict(h=bits(h), A=bits(A), B=bits(B), base=base, prior=prior, alpha=alpha, beta=beta,
                act=np.array(act), with_prior=np.array(with_prior), base_bf16=np.array(base_bf16),
                rank=bits(rank), ids=ids, score=score, second=second)


def gru_case(seed, nb, G, rows, bias):
    rng = np.random.default_rng(seed)
    table = bf16(rng, (rows, 3 * G))
    W_hh = bf16(rng, (3 * G, G), 0.1)
    b_hh = bf16(rng, (3 * G,), 0.1) if bias else np.zeros(0, np.float32)
    h = bf16(rng, (nb, G), 0.7)
    tokens = rng.integers(0, rows, nb).astype(np.int64)
    out = oracle.gru_cell(table[tokens], h, W_hh, b_hh if bias else None)
    out0 = oracle.gru_cell(table[tokens], np.zeros_like(h), W_hh, b_hh if bias else None)
    return dict(table=bits(table), W_hh=bits(W_hh), b_hh=bits(b_hh), h=bits(h), tokens=tokens,
                h_out=bits(out), h_out_zero=bits(out0))


def rollout_case(seed, nb, steps, V, E, G, r, act):
    rng = np.random.default_rng(seed)
    emb = bf16(rng, (V, E))
    W_ih = bf16(rng, (3 * G, E), 0.2)
    W_hh = bf16(rng, (3 * G, G), 0.2)
    A = bf16(rng, (r, G), 0.2)
    Bw = bf16(rng, (V, r), 0.2)
    base = oracle.bf16_round((rng.standard_normal((nb, steps, V)) * 3).astype(np.float32))
    prior = oracle.bf16_round(np.log(rng.dirichlet(np.ones(V))).astype(np.float32))
    alphas = rng.uniform(0, 0.6, steps).astype(np.float32)
    betas = rng.uniform(0, 0.6, steps).astype(np.float32)
    betas[1] = 0.0
    prefix = rng.integers(0, V, nb).astype(np.int64)
    gi_table = oracle.gru_input_table(emb, W_ih)
    ids, scores, seconds = oracle.rollout(prefix, base, gi_table=gi_table, W_hh=W_hh, b_hh=None, A=A,
                                          rank_bias=None, act=act, B=Bw, prior=prior, alphas=alphas,
                                          betas=betas)
    return dict(emb=bits(emb), W_ih=bits(W_ih), W_hh=bits(W_hh), A=bits(A), B=bits(Bw), base=bits(base),
                prior=bits(prior), alphas=alphas, betas=betas, prefix=prefix, act=np.array(act),
                gi_table=bits(gi_table), ids=ids, scores=scores, seconds=seconds)


CASES = {
    "argmax_ragged_silu_f32.npz": lambda: argmax_case(100, M=8, d=128, r=64, V=1031, act="silu",
                                                      base_bf16=False, with_prior=True, plant=True),
    "argmax_bf16_identity.npz": lambda: argmax_case(101, M=5, d=64, r=32, V=777, act="identity",
                                                    base_bf16=True, with_prior=True, plant=True),
    "argmax_noprior_m20.npz": lambda: argmax_case(102, M=20, d=64, r=96, V=600, act="identity",
                                                  base_bf16=False, with_prior=False, plant=False),
    "gru_b4_g32.npz": lambda: gru_case(103, nb=4, G=32, rows=40, bias=False),
    "gru_b17_g48_bias.npz": lambda: gru_case(104, nb=17, G=48, rows=30, bias=True),
    "rollout_b2_s6.npz": lambda: rollout_case(105, nb=2, steps=6, V=600, E=16, G=32, r=32, act="silu"),
}


def main():
    for name, make in CASES.items():
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **make())
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
