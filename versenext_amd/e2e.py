"""End-to-end speculative decoding on one MI355X: a draft model proposes k
tokens per sequence, the target verifies all k+1 positions in one
incremental forward, and the acceptance kernel commits a variable number of
tokens per sequence.

Per round (all sequences of the batch at once):
1. draft: k+1 one-token forwards of the draft at positions lens_d[b] + i
   (the last one only writes x_k into the draft's cache); q_i = draft logits
   (B, k, V) fp32 from the INT4 head GEMV; x_{i+1} drawn from
   softmax(q_i / T) (argmax when greedy);
2. verify: the target runs [c, x_1 .. x_k] at positions lens_t[b] + i and
   the matrix-core LM head writes p (B, k+1, V) fp32;
3. accept: vnx_spec_accept (Leviathan et al. 2023, Alg. 1 with host uniforms)
   or, greedy, vnx_greedy_verify with the bonus row: n_b accepted tokens and
   one drawn / bonus token per sequence;
4. commit: lens_t, lens_d += n_b + 1 (the rejected suffix of both caches is
   rolled back by not advancing), the drawn token becomes c.

The greedy rule is the reference's verify / verify_then_commit
(packages/verse_nex/verse_nex/speculative.py:168-310) for every batch row,
plus the bonus token when all k drafts match; the emitted stream equals the
target's greedy stream.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Optional

import torch

from .model import CometSparkGPU


@dataclass
class DecodeStats:
    rounds: int = 0
    emitted: int = 0                 # tokens committed (capped at n_new per row)
    accepted_drafts: int = 0         # draft tokens accepted (uncapped)
    decode_s: float = 0.0
    prefill_s: float = 0.0
    draft_s: float = 0.0             # host-timed phase split (with syncs), optional
    verify_s: float = 0.0
    accept_s: float = 0.0
    per_round_tokens: list = field(default_factory=list)

    @property
    def tokens_per_s(self) -> float:
        return self.emitted / self.decode_s if self.decode_s > 0 else 0.0


class SpecDecodeEngine:
    def __init__(self, target: CometSparkGPU, draft: CometSparkGPU, hip, k: int, temperature: float,
                 seed: int = 31):
        if target.B != draft.B:
            raise ValueError("target and draft caches must have the same batch")
        if target.cfg.vocab_size != draft.cfg.vocab_size:
            raise ValueError("target and draft must share the vocabulary")
        if k < 1:
            raise ValueError("k must be >= 1")
        self.t, self.d, self.hip = target, draft, hip
        self.k = int(k)
        self.T = float(temperature)
        self.greedy = self.T <= 0.0
        self.B = target.B
        self.V = target.cfg.vocab_size
        dev = hip.torch_device
        self.dev = dev
        self.gen = torch.Generator(device=dev)
        self.gen.manual_seed(int(seed))
        self.pbuf = torch.empty((self.B, self.k + 1, self.V), dtype=torch.float32, device=dev)
        self.qbuf = torch.empty((self.B, self.k, self.V), dtype=torch.float32, device=dev)

    # ---- phases ---------------------------------------------------------
    def _sample(self, logits: torch.Tensor) -> torch.Tensor:
        if self.greedy:
            return self.hip.argmax(logits).view(-1)
        probs = torch.softmax(logits / self.T, dim=-1)
        return torch.multinomial(probs, 1, generator=self.gen).view(-1)

    def _draft(self, c, lens_d, Tmax_d):
        B, k = self.B, self.k
        xs = torch.empty((B, k), dtype=torch.int64, device=self.dev)
        tok = c
        for i in range(k + 1):
            h = self.d.forward(tok.view(B, 1), lens_d + i, Tmax_d + i)
            if i == k:
                break
            self.qbuf[:, i] = self.d.logits(h).view(B, self.V)
            tok = self._sample(self.qbuf[:, i])
            xs[:, i] = tok
        return xs

    def _verify(self, c, xs, lens_t, Tmax_t):
        toks = torch.cat([c.view(self.B, 1), xs], dim=1)
        h = self.t.forward(toks, lens_t, Tmax_t)
        self.t.logits(h, out=self.pbuf)

    def _accept(self, xs):
        if self.greedy:
            _, _, alen, out = self.hip.greedy_verify(self.pbuf, xs, rows_t=self.k + 1)
            return alen, out
        u = torch.rand((self.B, self.k + 1), generator=self.gen, device=self.dev)
        res = self.hip.spec_accept(self.pbuf, self.qbuf, xs, u, temperature=self.T)
        return res["accept_len"], res["out_ids"]

    # ---- driver ---------------------------------------------------------
    @torch.no_grad()
    def generate(self, prompts: torch.Tensor, n_new: int, phase_timing: bool = False):
        """prompts (B, T0) int64 on the device.  Returns (tokens (B, n_new)
        int64 on the device, DecodeStats).  Prefill is timed separately from
        the decode rounds."""
        B, T0 = prompts.shape
        if B != self.B:
            raise ValueError(f"batch {B} != {self.B}")
        k = self.k
        dev = self.dev
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        lens_t = torch.zeros(B, dtype=torch.int32, device=dev)
        lens_d = torch.zeros(B, dtype=torch.int32, device=dev)
        if T0 > 1:
            self.t.forward(prompts[:, :-1], lens_t, 0)
            self.d.forward(prompts[:, :-1], lens_d, 0)
        lens_t += T0 - 1
        lens_d += T0 - 1
        c = prompts[:, -1].clone()
        torch.cuda.synchronize(dev)
        st = DecodeStats(prefill_s=time.perf_counter() - t0)

        out = torch.full((B, n_new + k + 1), -1, dtype=torch.int64, device=dev)
        count = torch.zeros(B, dtype=torch.int64, device=dev)
        ar = torch.arange(k + 1, device=dev).view(1, k + 1)
        bidx = torch.arange(B, device=dev).view(B, 1).expand(B, k + 1)
        Tmax_t = Tmax_d = T0 - 1
        t1 = time.perf_counter()
        while True:
            ta = time.perf_counter()
            xs = self._draft(c, lens_d, Tmax_d)
            if phase_timing:
                torch.cuda.synchronize(dev)
            tb = time.perf_counter()
            self._verify(c, xs, lens_t, Tmax_t)
            if phase_timing:
                torch.cuda.synchronize(dev)
            tc = time.perf_counter()
            alen, ids = self._accept(xs)
            n1 = alen.long() + 1                                     # tokens committed this round
            keep = ar < n1.view(B, 1)
            pos = (count.view(B, 1) + ar).clamp(max=n_new + k)
            out[bidx[keep], pos[keep]] = ids[keep]
            count += n1
            c = ids.gather(1, alen.long().view(B, 1)).view(B)
            lens_t += n1.int()
            lens_d += n1.int()
            info = torch.stack([count.min(), lens_t.max().long(), lens_d.max().long(), alen.long().sum()]).cpu()
            st.rounds += 1
            st.per_round_tokens.append(int(info[3]) + B)
            if phase_timing:
                td = time.perf_counter()
                st.draft_s += tb - ta
                st.verify_s += tc - tb
                st.accept_s += td - tc
            if int(info[0]) >= n_new:
                break
            Tmax_t, Tmax_d = int(info[1]), int(info[2])
            if Tmax_t + k + 1 > self.t.cap or Tmax_d + k + 1 > self.d.cap:
                raise RuntimeError("KV cache capacity exhausted")
        torch.cuda.synchronize(dev)
        st.decode_s = time.perf_counter() - t1
        st.emitted = B * n_new
        st.accepted_drafts = sum(st.per_round_tokens) - B * st.rounds
        return out[:, :n_new], st
