"""Seeded synthetic inputs for the acceptance tests (BASELINE.json config 2 recipe):
target logits ~ N(0, 2) (default_rng(seed_t)), draft = target[:, :k] + N(0, 0.5)
(default_rng(seed_d)), draft ids drawn from q_i by inverse CDF with
default_rng(seed_x) uniforms, acceptance uniforms default_rng(seed_u)."""
import numpy as np

from oracle import _clib, rows


def make_inputs(B, k, V, T=0.8, seed_t=0, seed_d=2, seed_x=3, seed_u=1, sigma=2.0, noise=0.5):
    tgt = np.random.default_rng(seed_t).normal(0.0, sigma, (B, k + 1, V)).astype(np.float32)
    dft = (tgt[:, :k] + np.random.default_rng(seed_d).normal(0.0, noise, (B, k, V))).astype(np.float32)
    ux = np.random.default_rng(seed_x).random((B, k)).astype(np.float32)
    ids = np.empty((B, k), np.int64)
    for b in range(B):
        a = rows.scale(dft[b], T)
        L = rows.lse64(a).astype(np.float32)
        for i in range(k):
            w = _clib.exp_canon(a[i] - L[i])
            ids[b, i] = _clib.icdf(w, ux[b, i])[0]
    u = np.random.default_rng(seed_u).random((B, k + 1)).astype(np.float32)
    return tgt, dft, ids, u
