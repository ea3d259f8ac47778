"""Speculative-decoding verification oracles (test infrastructure only).

1. `RefSpeculativeDecoder`: the reference's greedy Medusa verifier restated in
   numpy (packages/verse_nex/verse_nex/speculative.py): draft heads + argmax
   (:101-104, :110-162), verify (:168-224), verify_then_commit (:230-310).
   Pinned by the reference's own test vectors (tests/test_speculative_decode.py),
   re-run against this restatement in tests/test_oracle_speculative.py.

2. `greedy_verify_batched`: verify + the commit prefix rule for every batch row
   (the reference handles row 0 only, speculative.py:262-268), optionally with
   a bonus row.  Pinned by (1) on row 0 and by brute force.

3. `spec_accept`: the stochastic acceptance rule of Leviathan, Kalman & Matias
   2023 (arXiv:2211.17192, Alg. 1) / Chen et al. 2023 (arXiv:2302.01318) with
   explicit uniforms, in the exact arithmetic the kernels use:
     a = RN(l / T) (sampler.py:95), masked below the top-k threshold;
     L32 = RN32(log sum exp a) with the LSE in fp64;
     p(x) = E(a_x - L32_p), q(x) = E(b_x - L32_q), E = canonical exp (canon.c);
     accept i  iff  u_i < 1 and u_i * q(x_i) < p(x_i)   (u < min(1, p/q));
     n = first rejection; emitted token at n = inverse-CDF draw with u_k from
     max(0, p_n - q_n) (n < k; from p_n if that mass is 0) or from p_k (n = k).
   No reference implementation exists (the reference verifier is greedy).
   Pinned by: the T -> 0 limit equal to (2) with a bonus row; p == q accepts
   all; p(x) = 0 rejects; the exact output law equals p (unbiasedness
   theorem) on exhaustive u-grids for small V; icdf equal to numpy's
   Generator.choice on the same underlying uniform.
"""
from __future__ import annotations

import numpy as np

from . import _clib, rows

FLAG_NEAR_TIE = 1
FLAG_LSE_EDGE = 2
FLAG_CDF_EDGE = 4
FLAG_ZERO_RESIDUAL = 8
FLAG_BAD_ID = 16


def _data(x):
    """numpy view of an ndarray / verse_torch-like Tensor (has .data) / torch tensor."""
    if hasattr(x, "detach") and hasattr(x, "cpu"):
        return x.detach().cpu().numpy()
    if isinstance(x, np.ndarray):
        return x
    if hasattr(x, "data"):
        return _data(x.data)
    return np.asarray(x)


class RefSpeculativeDecoder:
    """Greedy Medusa verifier, restated from speculative.py:55-310 (numpy only)."""

    def __init__(self, dim: int, vocab_size: int, num_draft_heads: int = 4, seed: int | None = None):
        if num_draft_heads < 1:
            raise ValueError(f"num_draft_heads must be >= 1, got {num_draft_heads}")
        self.dim = int(dim)
        self.vocab_size = int(vocab_size)
        self.num_draft_heads = int(num_draft_heads)
        rng = np.random.default_rng(seed)
        bound = 1.0 / np.sqrt(self.dim)
        # Linear(dim, vocab, bias=False): weight (vocab, dim), y = x @ W.T (vnnn.py:394-430)
        self.head_weights = [rng.uniform(-bound, bound, (self.vocab_size, self.dim)).astype(np.float32)
                             for _ in range(self.num_draft_heads)]

    def draft(self, hidden):
        h = np.asarray(_data(hidden), dtype=np.float32)
        if h.ndim == 2:
            h = h[:, None, :]
        elif h.ndim == 3:
            h = h[:, -1:, :]
        elif h.ndim == 4:
            h = h.reshape(h.shape[0], -1, h.shape[-1])[:, -1:, :]
        else:
            raise ValueError(f"hidden ndim {h.ndim} unsupported, expected 2/3/4")
        logits_list, toks = [], []
        for W in self.head_weights:
            lg = (h @ W.T)[:, 0, :]
            logits_list.append(lg)
            toks.append(np.argmax(lg, axis=-1))
        return np.stack(toks, axis=1).astype(np.int64), logits_list

    def verify(self, draft_tokens, main_model, context_tokens):
        draft_tokens = np.asarray(draft_tokens)
        context_tokens = np.asarray(context_tokens)
        if draft_tokens.ndim != 2 or context_tokens.ndim != 2:
            raise ValueError("draft_tokens / context_tokens must be 2-D")
        if draft_tokens.shape[0] != context_tokens.shape[0]:
            raise ValueError("batch mismatch")
        B, k = draft_tokens.shape
        T_ctx = context_tokens.shape[1]
        full = np.concatenate([context_tokens, draft_tokens], axis=1).astype(np.int64)
        out = main_model(full)
        logits = out[0] if isinstance(out, tuple) else out
        logits_np = np.asarray(_data(logits))
        start = T_ctx - 1
        main_pred = np.argmax(logits_np[:, start:start + k, :], axis=-1)
        return draft_tokens == main_pred, main_pred

    def verify_then_commit(self, draft_tokens, main_model, context_tokens, max_redraft_rounds: int = 1):
        draft_tokens = np.asarray(draft_tokens)
        context_tokens = np.asarray(context_tokens)
        B, k = draft_tokens.shape
        d_b, c_b = draft_tokens[:1], context_tokens[:1]
        acc_mask, main_pred = self.verify(d_b, main_model, c_b)
        accepted, all_ok = [], True
        for i in range(k):
            if acc_mask[0, i]:
                accepted.append(int(d_b[0, i]))
            else:
                accepted.append(int(main_pred[0, i]))
                all_ok = False
                break
        new_ctx = np.concatenate([c_b, np.asarray(accepted, dtype=np.int64)[None, :]], axis=1)
        if not all_ok and max_redraft_rounds > 0:
            out = main_model(new_ctx.astype(np.int64))
            hid = (out[1] if len(out) > 1 else out[0]) if isinstance(out, tuple) else out
            self.draft(hid)
        return accepted, all_ok, new_ctx


def greedy_verify_batched(target: np.ndarray, draft_ids: np.ndarray):
    """target (B, rows_t, V) with rows_t in {k, k+1}; returns
    (accepted (B,k) bool, main_pred (B,rows_t), accept_len (B,), out_ids (B,k+1))."""
    target = np.asarray(target)
    ids = np.asarray(draft_ids, dtype=np.int64)
    B, rows_t, V = target.shape
    k = ids.shape[1]
    assert rows_t in (k, k + 1)
    pred = np.argmax(target, axis=-1).astype(np.int64)
    acc = ids == pred[:, :k]
    alen = np.zeros(B, np.int32)
    out = np.full((B, k + 1), -1, np.int64)
    for b in range(B):
        n = 0
        while n < k and acc[b, n]:
            n += 1
        alen[b] = n
        out[b, :n] = ids[b, :n]
        if n < k:
            out[b, n] = pred[b, n]
        elif rows_t == k + 1:
            out[b, k] = pred[b, k]
    return acc, pred, alen, out


def _near_f32_edge(L64: np.ndarray, L32: np.ndarray, tol: float) -> np.ndarray:
    up = np.nextafter(L32, np.float32(np.inf)).astype(np.float64)
    dn = np.nextafter(L32, np.float32(-np.inf)).astype(np.float64)
    mu = 0.5 * (L32.astype(np.float64) + up)
    md = 0.5 * (L32.astype(np.float64) + dn)
    with np.errstate(invalid="ignore"):
        near = (np.abs(L64 - mu) < tol) | (np.abs(L64 - md) < tol)
    return near & np.isfinite(L64)


def spec_accept(target, draft, draft_ids, uniforms, temperature, thr_t=None, thr_d=None,
                lse_edge_tol: float = 1e-7, cdf_edge_rel: float = 1e-12):
    """Canonical stochastic acceptance. target (B,k+1,V) f32, draft (B,k,V) f32,
    draft_ids (B,k) int64, uniforms (B,k+1) f32.  Returns a dict with
    accept_len (B,) int32, out_ids (B,k+1) int64, flags (B,k+1) uint8,
    lse_t (B,k+1) f32, lse_d (B,k) f32, lse_t64 / lse_d64 (fp64)."""
    target = np.asarray(target, dtype=np.float32)
    draft = np.asarray(draft, dtype=np.float32)
    ids = np.asarray(draft_ids, dtype=np.int64)
    u = np.asarray(uniforms, dtype=np.float32)
    B, K1, V = target.shape
    k = K1 - 1
    assert draft.shape == (B, k, V) and ids.shape == (B, k) and u.shape == (B, k + 1)
    T = np.float32(temperature)
    thr_t_a = np.full((B, k + 1), -np.inf, np.float32) if thr_t is None else np.asarray(thr_t, np.float32)
    thr_d_a = np.full((B, k), -np.inf, np.float32) if thr_d is None else np.asarray(thr_d, np.float32)

    lse_t64 = np.empty((B, k + 1))
    lse_d64 = np.empty((B, k))
    for b in range(B):  # row by row keeps the fp64 temporaries small
        lse_t64[b] = rows.lse64(rows.apply_threshold(rows.scale(target[b], T), thr_t_a[b]))
        lse_d64[b] = rows.lse64(rows.apply_threshold(rows.scale(draft[b], T), thr_d_a[b]))
    lse_t = lse_t64.astype(np.float32)
    lse_d = lse_d64.astype(np.float32)
    edge_t = _near_f32_edge(lse_t64, lse_t, lse_edge_tol)
    edge_d = _near_f32_edge(lse_d64, lse_d, lse_edge_tol)

    accept_len = np.zeros(B, np.int32)
    out = np.full((B, k + 1), -1, np.int64)
    flags = np.zeros((B, k + 1), np.uint8)
    for b in range(B):
        acc = np.zeros(k, bool)
        for i in range(k):
            x = int(ids[b, i])
            if 0 <= x < V:
                a = rows.scale(target[b, i, x:x + 1], T)[0]
                a = a if a >= thr_t_a[b, i] else np.float32(-np.inf)
                bq = rows.scale(draft[b, i, x:x + 1], T)[0]
                bq = bq if bq >= thr_d_a[b, i] else np.float32(-np.inf)
                pp = _clib.exp_canon(np.float32(a - lse_t[b, i]))[()]
                qq = _clib.exp_canon(np.float32(bq - lse_d[b, i]))[()]
                acc[i] = bool(u[b, i] < np.float32(1.0)) and (
                    np.float64(u[b, i]) * np.float64(qq) < np.float64(pp))
                if qq > 0:
                    ratio = min(1.0, float(pp) / float(qq))
                    if abs(float(u[b, i]) - ratio) < 1e-6:
                        flags[b, i] |= FLAG_NEAR_TIE
            else:
                flags[b, i] |= FLAG_BAD_ID
            if edge_t[b, i] or edge_d[b, i]:
                flags[b, i] |= FLAG_LSE_EDGE
        if edge_t[b, k]:
            flags[b, k] |= FLAG_LSE_EDGE
        n = 0
        while n < k and acc[n]:
            n += 1
        accept_len[b] = n
        out[b, :n] = ids[b, :n]
        if n < k:
            w_r, w_p = _clib.resid_weights(target[b, n], draft[b, n], T, thr_t_a[b, n], thr_d_a[b, n],
                                           lse_t[b, n], lse_d[b, n])
            j, before, after, total = _clib.icdf(w_r, u[b, k])
            if j < 0:
                flags[b, n] |= FLAG_ZERO_RESIDUAL
                j, before, after, total = _clib.icdf(w_p, u[b, k])
        else:
            w_r, _ = _clib.resid_weights(target[b, k], None, T, thr_t_a[b, k], -np.inf, lse_t[b, k], 0.0)
            j, before, after, total = _clib.icdf(w_r, u[b, k])
        if j < 0:
            flags[b, n] |= FLAG_ZERO_RESIDUAL
            j = 0
        else:
            target_mass = float(u[b, k]) * total
            if target_mass - before < cdf_edge_rel * total or after - target_mass < cdf_edge_rel * total:
                flags[b, n] |= FLAG_CDF_EDGE
        out[b, n] = j
    return dict(accept_len=accept_len, out_ids=out, flags=flags, lse_t=lse_t, lse_d=lse_d,
                lse_t64=lse_t64, lse_d64=lse_d64)


def output_law_on_grid(p_logits, q_logits, x_draft_probs, temperature, grid: int = 4096):
    """Exact output law of `spec_accept` for k = 1 on a midpoint u-grid.

    For every draft token x (weighted by x_draft_probs[x]) and every grid value
    of u_0 and u_1, runs the canonical rule and accumulates the law of the
    first emitted token.  By the unbiasedness theorem it must equal p_0."""
    p_logits = np.asarray(p_logits, np.float32)  # (2, V): rows 0 (position 0) and 1 (bonus)
    q_logits = np.asarray(q_logits, np.float32)  # (1, V)
    V = p_logits.shape[-1]
    us = ((np.arange(grid) + 0.5) / grid).astype(np.float32)
    law = np.zeros(V)
    for x in range(V):
        wx = float(x_draft_probs[x])
        if wx == 0.0:
            continue
        # acceptance probability over the u_0 grid
        res = spec_accept(p_logits[None], q_logits[None], np.array([[x]]),
                          np.array([[0.5, 0.5]], np.float32), temperature)
        L_p, L_q = res["lse_t"][0, 0], res["lse_d"][0, 0]
        a = rows.scale(p_logits[0, x:x + 1], temperature)[0]
        bq = rows.scale(q_logits[0, x:x + 1], temperature)[0]
        pp = float(_clib.exp_canon(np.float32(a - L_p)))
        qq = float(_clib.exp_canon(np.float32(bq - L_q)))
        acc_frac = float(np.mean([(u < 1.0) and (float(u) * qq < pp) for u in us]))
        law[x] += wx * acc_frac
        w_r, w_p = _clib.resid_weights(p_logits[0], q_logits[0], temperature, -np.inf, -np.inf, L_p, L_q)
        w = w_r if float(np.sum(w_r, dtype=np.float64)) > 0 else w_p
        hits = np.zeros(V)
        for u in us:
            j, _, _, _ = _clib.icdf(w, u)
            hits[j] += 1
        law += wx * (1.0 - acc_frac) * hits / grid
    return law
