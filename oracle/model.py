"""CPU restatement of the CometSpark (VerseNex) language-model forward pass
(test infrastructure only: the checker of versenext_amd/model.py, and the
reference CPU path timed beside it).

numpy float32, the whole sequence in parallel with no KV cache, the way the
reference's verifier calls the model (speculative.py:202-213):
- CometSparkV05LM.forward (spark/src/base_model.py:170-208): tok_emb(idx) x
  sqrt(D), the blocks, the final RMSNorm, the tied head x @ tok_emb^T;
- VerseNexBlock.forward (packages/verse_nex/verse_nex/cometspark.py:209-247);
- RMSNorm (packages/verse_torch/verse_torch/vnnn.py:593-615 via
  _normalize_kernel :468-508): x / sqrt(mean(x*x) + eps) * w;
- TriSparseAttention.forward (packages/verse_nex/verse_nex/tri_sparse_attn.py
  :536-613): projections, RoPE (:167-221), repeat_kv adjacent copies,
  sliding-window path (:260-400; written here as one masked softmax over the
  window, which the chunked form equals: tests/test_oracle_swa_replay.py
  replays the reference's parallel-vs-serial cases against it), global path
  (:469-495), ALiBi path when use_alibi and T <= 1024 (:501-534), sigmoid
  gates (:585-608);
- SwiGLUMLP (vnnn.py:779-807); MoDLayer / DensePart / Router / Expert
  (packages/verse_nex/verse_nex/mod.py:142-213, :337-440, :466-803):
  argsort(-logits)[:k] selection, softmax over the selected logits.

Pinned by tests/test_oracle_model.py against golden vectors written by the
reference itself (tests/golden/make_cometspark_small.py): the logits of the
config-1 target for a 16-token prompt and its 128-token greedy stream.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


def _rms(x, w, eps):
    ms = (x * x).mean(axis=-1, keepdims=True)
    return (x / np.sqrt(ms + F32(eps))) * w


def _softmax(x, axis=-1):
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def _sigmoid(x):
    return F32(1.0) / (F32(1.0) + np.exp(-x))


def _silu(x):
    return x * _sigmoid(x)


def rope_tables(d, T, theta):
    half = d // 2
    i = np.arange(half, dtype=F32)
    inv_freq = F32(1.0) / (F32(theta) ** (F32(2.0) * i / F32(d)))
    ang = np.outer(np.arange(T, dtype=F32), inv_freq).astype(F32)
    cos = np.concatenate([np.cos(ang), np.cos(ang)], axis=-1).astype(F32)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], axis=-1).astype(F32)
    return cos, sin


def _rope(x, cos, sin):
    """x (B, T, heads, d); rotate_half = concat(-x[half:], x[:half])."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos[None, :, None, :] + rot * sin[None, :, None, :]


def _attend(q, k, v, bias):
    """softmax(q k^T / sqrt(d) + bias) v over (B, H, Tq, d) x (B|1, H, Tk, d)."""
    scale = 1.0 / (q.shape[-1] ** 0.5)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    if bias is not None:
        s = s + bias
    return _softmax(s) @ v


def alibi_slopes(H):
    """m_h = 1 / 2^(h / H), h = 1..H (tri_sparse_attn.py:151-155)."""
    return (1.0 / (2.0 ** (np.arange(1, H + 1, dtype=F32) / H))).astype(F32)


def swa_attention(q, k, v, window, offset=0):
    """Path A (tri_sparse_attn.py:258-448) as one masked softmax: queries at
    positions offset + i, keys at 0 .. Tk-1, key j visible iff j <= pos and
    pos - j < window; masked scores get -1e9.  (B, H, Tq, d)."""
    Tq, Tk = q.shape[2], k.shape[2]
    i = np.arange(Tq)[:, None] + offset
    j = np.arange(Tk)[None, :]
    ok = (j <= i) & ((i - j) < window)
    return _attend(q, k, v, np.where(ok, F32(0.0), F32(-1e9)).astype(F32)[None, None])


def alibi_attention(q, k, v, slopes, offset=0):
    """Path C (tri_sparse_attn.py:501-534): causal, bias -m_h * (pos - j)."""
    Tq, Tk = q.shape[2], k.shape[2]
    i = np.arange(Tq)[:, None] + offset
    j = np.arange(Tk)[None, :]
    dist = (i - j).astype(F32)
    bias = np.where((j <= i)[None], -slopes[:, None, None] * dist[None], F32(-1e9)).astype(F32)
    return _attend(q, k, v, bias[None])


def trisparse_heads(q, k, v, kg, vg, gate, cfg, offset=0):
    """The gated paths before the output projection (tri_sparse_attn.py:
    585-608): q (B, H, Tq, d); k, v (B, H, Tk, d) after repeat_kv; kg, vg the
    global rows (1, H, G, d); gate = sigmoid(gate_logits)."""
    out = gate[0] * swa_attention(q, k, v, cfg.window_size, offset) + gate[1] * _attend(q, kg, vg, None)
    if cfg.use_alibi and k.shape[2] <= 1024:
        out = out + gate[2] * alibi_attention(q, k, v, alibi_slopes(q.shape[1]), offset)
    return out


def trisparse(W, p, cfg, x):
    B, T, D = x.shape
    H, Hkv = cfg.n_head, cfg.n_kv_head
    d = D // H
    rep = H // Hkv
    q = (x @ W[p + "attn.wq.weight"].T).reshape(B, T, H, d)
    k = (x @ W[p + "attn.wk.weight"].T).reshape(B, T, Hkv, d)
    v = (x @ W[p + "attn.wv.weight"].T).reshape(B, T, Hkv, d)
    if cfg.use_rope:
        cos, sin = rope_tables(d, T, cfg.rope_theta)
        q, k = _rope(q, cos, sin), _rope(k, cos, sin)
    k = np.repeat(k, rep, axis=2).transpose(0, 2, 1, 3)
    v = np.repeat(v, rep, axis=2).transpose(0, 2, 1, 3)
    q = q.transpose(0, 2, 1, 3)
    g = W[p + "attn.global_tokens.weight"]
    G = g.shape[0]
    kg = np.repeat((g @ W[p + "attn.wk.weight"].T).reshape(1, G, Hkv, d), rep, axis=2).transpose(0, 2, 1, 3)
    vg = np.repeat((g @ W[p + "attn.wv.weight"].T).reshape(1, G, Hkv, d), rep, axis=2).transpose(0, 2, 1, 3)
    gate = _sigmoid(W[p + "attn.gate_logits"].astype(F32))
    out = trisparse_heads(q, k, v, kg, vg, gate, cfg)
    out = out.transpose(0, 2, 1, 3).reshape(B, T, H * d)
    return out @ W[p + "attn.proj.weight"].T


def swiglu(x, wg, wu, wd):
    return (_silu(x @ wg.T) * (x @ wu.T)) @ wd.T


def _route(logits, k):
    """argsort(-logits)[..., :k] and the softmax over the selected logits
    (Router.forward, mod.py:337-440)."""
    idx = np.argsort(-logits, axis=-1)[..., :k]
    sel = np.take_along_axis(logits, idx, axis=-1)
    return idx, _softmax(sel)


def mod(W, p, cfg, x):
    P, E, k = cfg.num_dense_parts, cfg.num_experts_per_part, cfg.top_k
    pidx, pw = _route(x @ W[p + "ffn.part_router.gate.weight"].T, P)
    out = np.zeros_like(x)
    for q in range(P):
        part_w = (pw * (pidx == q)).sum(axis=-1, keepdims=True)
        rp = p + f"ffn.parts.{q}."
        eidx, ew = _route(x @ W[rp + "router.gate.weight"].T, k)
        comb = np.zeros_like(x)
        for e in range(E):
            we = (ew * (eidx == e)).sum(axis=-1)
            mask = (eidx == e).any(axis=-1)
            if not mask.any():
                continue
            ep = rp + f"experts.{e}."
            ye = swiglu(x[mask], W[ep + "w_gate.weight"], W[ep + "w_up.weight"], W[ep + "w_down.weight"])
            add = np.zeros_like(x)
            add[mask] = ye * we[mask][:, None]
            comb = comb + add
        out = out + comb * part_w
    return out


def forward(W, cfg, idx, return_hidden=False, last_n=None, head=None):
    """logits (B, T, V) float32 of the tokens idx (B, T); with last_n, only
    the last last_n positions go through the head (the verifier reads k+1
    rows, speculative.py:218-220).  head: the (V, D) head weight when it is
    stored apart from the input embedding (a quantized copy of the tied
    table); else W['head.weight'] for an untied model (cfg.tie_weights
    False), else the tied table itself (cometspark.py:396-398)."""
    idx = np.asarray(idx, dtype=np.int64)
    if idx.ndim == 1:
        idx = idx[None]
    emb = W["tok_emb.weight"]
    x = emb[idx].astype(F32)
    if cfg.embedding_scale:
        x = x * math.sqrt(cfg.dim)
    x = x.astype(F32)
    for i, kind in enumerate(cfg.layer_pattern):
        p = f"blocks.{i}."
        x = x + trisparse(W, p, cfg, _rms(x, W[p + "norm1.weight"], cfg.eps))
        h = _rms(x, W[p + "norm2.weight"], cfg.eps)
        if kind == "mod":
            x = x + mod(W, p, cfg, h)
        else:
            x = x + swiglu(h, W[p + "ffn.w_gate.weight"], W[p + "ffn.w_up.weight"], W[p + "ffn.w_down.weight"])
    x = _rms(x, W["norm.weight"], cfg.eps)
    if return_hidden:
        return x
    if last_n is not None:
        x = x[:, -last_n:]
    if head is None and not getattr(cfg, "tie_weights", True):
        head = W["head.weight"]
    return x @ (emb if head is None else head).T


def _row_chunks(n_rows: int, rows: int):
    return [(i, min(n_rows, i + rows)) for i in range(0, n_rows, rows)]


def _threads() -> int:
    import os
    return max(1, min(16, os.cpu_count() or 1))


def _parallel_rows(fn, a, out, rows: int = 4096):
    """out[i:j] = fn(a[i:j]) over row chunks of a 2-D array, on a thread pool
    (numpy's ufuncs release the GIL); the result is the same as one call."""
    from concurrent.futures import ThreadPoolExecutor
    chunks = _row_chunks(a.shape[0], rows)
    if len(chunks) == 1:
        out[...] = fn(a)
        return out

    def one(c):
        out[c[0]:c[1]] = fn(a[c[0]:c[1]])
    with ThreadPoolExecutor(max_workers=_threads()) as ex:
        list(ex.map(one, chunks))
    return out


def _bf16_round_block(a):
    u = a.view(np.uint32)
    # finite values and infinities cannot overflow uint32 here (the largest,
    # 0xFF800000, plus 0x8000 stays below 2^32); NaNs are restored below
    r = u + np.uint32(0x7FFF)
    r += (u >> np.uint32(16)) & np.uint32(1)
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, a, out)
    return out


def bf16_round(a):
    """float32 values rounded to bfloat16 (round to nearest, ties to even),
    returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if a.ndim < 2:
        return _bf16_round_block(a.reshape(1, -1)).reshape(a.shape).astype(np.float32)
    flat = a.reshape(a.shape[0], -1)
    out = np.empty_like(flat)
    _parallel_rows(_bf16_round_block, flat, out)
    return out.reshape(a.shape)


_MATRICES = ("attn.wq.weight", "attn.wk.weight", "attn.wv.weight", "attn.proj.weight", "w_gate.weight",
             "w_up.weight", "w_down.weight")


def int4_g_stored(w, group: int = 128):
    """The exact dequantization q * s of the INT4 group quantization of w
    (oracle.quant.quantize_int4_g then dequantize_int4_g, applied to row
    chunks on a thread pool: both are row-local)."""
    from . import quant as OQ
    w = np.ascontiguousarray(w, dtype=np.float32)

    def rt(c):
        q, s = OQ.quantize_int4_g(c, group)
        return OQ.dequantize_int4_g(q, s, c.shape, group)
    return _parallel_rows(rt, w, np.empty_like(w), rows=2048)


def stored_weights(W, int4: bool = False):
    """The weights a GPU model holds, restated for this forward
    (versenext_amd/model.py CometSparkGPU): every projection matrix and the
    embedding table rounded to bfloat16; with int4, the projection matrices
    are instead the exact dequantization q * s of their INT4 group-128
    quantization (oracle.quant.quantize_int4_g) and the head is the
    dequantized INT4 copy of the embedding table (returned second, else
    None).  Norm weights, router weights, global tokens and gate logits stay
    float32."""
    out = {}
    for k, v in W.items():
        v = np.asarray(v, np.float32)
        if k.endswith(_MATRICES):
            if int4 and v.shape[1] % 128 == 0:
                out[k] = int4_g_stored(v, 128)
            else:
                out[k] = bf16_round(v)
        elif k == "tok_emb.weight":
            out[k] = bf16_round(v)
        else:
            out[k] = v
    head = None
    if int4:
        head = int4_g_stored(np.asarray(W["tok_emb.weight"], np.float32), 128)
    return out, head


def greedy_stream(W, cfg, prompt, n_new):
    """The target's greedy continuation with a full re-forward per token (the
    stream greedy speculative decoding reproduces, speculative.py:22)."""
    seq = list(np.asarray(prompt, dtype=np.int64).reshape(-1))
    out = []
    for _ in range(n_new):
        logits = forward(W, cfg, np.asarray(seq)[None])[0, -1]
        t = int(np.argmax(logits))
        out.append(t)
        seq.append(t)
    return np.asarray(out, dtype=np.int64)


def spec_decode_greedy(Wt, cfg_t, Wd, cfg_d, prompt, n_new, k):
    """The reference's greedy speculative decode, batch row 0
    (SpeculativeDecoder.verify_then_commit, speculative.py:230-310): the draft
    model proposes k tokens by greedy argmax (re-forwarding its context), the
    target re-forwards [context, draft] and the longest prefix agreeing with
    its argmax is committed plus the target's token at the first mismatch
    (no bonus token when all k agree).  Returns (tokens, steps)."""
    seq = list(np.asarray(prompt, dtype=np.int64).reshape(-1))
    out = []
    steps = 0
    while len(out) < n_new:
        ctx = list(seq)
        draft = []
        for _ in range(k):
            t = int(np.argmax(forward(Wd, cfg_d, np.asarray(ctx)[None])[0, -1]))
            draft.append(t)
            ctx.append(t)
        T = len(seq)
        logits = forward(Wt, cfg_t, np.asarray(seq + draft)[None])[0]
        pred = np.argmax(logits[T - 1:T - 1 + k], axis=-1)
        n = 0
        while n < k and draft[n] == int(pred[n]):
            n += 1
        acc = draft[:n] if n == k else draft[:n] + [int(pred[n])]
        steps += 1
        for t in acc:
            if len(out) < n_new:
                out.append(t)
                seq.append(t)
    return np.asarray(out, dtype=np.int64), steps


def spec_round_cpu(Wt, cfg_t, Wd, cfg_d, seq, k, temperature, u_draft, u_acc):
    """One stochastic speculative round for one sequence on the CPU, the
    reference's way (full re-forward, no KV cache, speculative.py:202-213):
    k draft tokens drawn from softmax(draft logits / T) with u_draft[i]
    (inverse CDF, the acceptance kernels' draw), one target re-forward of
    [seq, drafts] read at the k+1 verified positions, then the canonical
    acceptance (oracle.speculative.spec_accept) with u_acc.  Returns the
    committed tokens (accepted drafts + the drawn / bonus token)."""
    from .speculative import spec_accept
    ctx = list(np.asarray(seq, dtype=np.int64).reshape(-1))
    V = cfg_t.vocab_size
    q = np.empty((1, k, V), np.float32)
    xs = []
    empty_d = np.zeros((1, 0, V), np.float32)
    empty_i = np.zeros((1, 0), np.int64)
    for i in range(k):
        q[0, i] = forward(Wd, cfg_d, np.asarray(ctx)[None], last_n=1)[0, -1]
        r = spec_accept(q[:, i:i + 1], empty_d, empty_i, np.asarray([[u_draft[i]]], np.float32), temperature)
        x = int(r["out_ids"][0, 0])
        xs.append(x)
        ctx.append(x)
    p = forward(Wt, cfg_t, np.asarray(ctx)[None], last_n=k + 1)
    res = spec_accept(p, q, np.asarray([xs], np.int64), np.asarray(u_acc, np.float32).reshape(1, k + 1),
                      temperature)
    n = int(res["accept_len"][0])
    return [int(t) for t in res["out_ids"][0, :n + 1]]
