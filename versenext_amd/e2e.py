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
3. accept: vnx_spec_accept_draft_lse (Leviathan et al. 2023, Alg. 1 with
   host uniforms; the draft rows' LSEs come from the draws of step 1) or,
   greedy, vnx_greedy_verify with the bonus row: n_b accepted tokens and
   one drawn / bonus token per sequence;
4. commit: lens_t, lens_d += n_b + 1 (the rejected suffix of both caches is
   rolled back by not advancing), the drawn token becomes c.

The greedy rule is the reference's verify / verify_then_commit
(packages/verse_nex/verse_nex/speculative.py:168-310) for every batch row,
plus the bonus token when all k drafts match; the emitted stream equals the
target's greedy stream.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib
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
    """One round = draft (k+1 one-token forwards + k draws), verify (one
    (k+1)-token target forward + LM head), accept, commit; every round works
    on the engine's static device buffers, so the whole round can be
    captured once as a HIP graph (use_graph) and replayed: the uniforms of a
    round are drawn into their buffers before each replay, and the attention
    calls take the cache bound as their prefix maximum (each row reads only
    its own lens[b] prefix rows)."""

    def __init__(self, target: CometSparkGPU, draft: CometSparkGPU, hip, k: int, temperature: float,
                 seed: int = 31, use_graph: bool = False, logits_dtype: Optional[torch.dtype] = None):
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
        self.use_graph = bool(use_graph)
        dev = hip.torch_device
        self.dev = dev
        self.gen = torch.Generator(device=dev)
        self.gen.manual_seed(int(seed))
        B, k = self.B, self.k
        # Logits of a sampled round stay in a bf16 target's dtype (the
        # reference's head Linear returns them in the module dtype,
        # spark/src/base_model.py:207): half the bytes for the heads to write
        # and the draws and the acceptance to read.  Greedy rounds, fp32
        # models and heads without a bf16 output keep fp32.
        if logits_dtype is None:
            logits_dtype = (torch.bfloat16 if not self.greedy and target.dtype == torch.bfloat16
                            and target.head_writes_bf16() and draft.head_writes_bf16() else torch.float32)
        if logits_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("logits_dtype must be torch.float32 or torch.bfloat16")
        self.logits_dtype = logits_dtype
        self.pbuf = torch.empty((B, k + 1, self.V), dtype=logits_dtype, device=dev)
        self.qbuf = torch.empty((B, k, self.V), dtype=logits_dtype, device=dev)
        # both uniform arrays in one buffer (u_acc at a 256-byte boundary), so
        # a round's fill is one launch
        off = (k * B + 63) // 64 * 64
        self.u_all = torch.zeros(off + B * (k + 1), dtype=torch.float32, device=dev)
        self.u_draft = self.u_all[:k * B].view(k, B)
        self.u_acc = self.u_all[off:].view(B, k + 1)
        self.xsT = torch.zeros((k, B), dtype=torch.int64, device=dev)   # draft token i of every row: xsT[i]
        # the draws' row LSEs of q_i / T and their flags, which the acceptance
        # takes instead of streaming the k draft rows again
        self.lse_dr = torch.zeros((k, B), dtype=torch.float32, device=dev)
        self.fl_dr = torch.zeros((k, B), dtype=torch.uint8, device=dev)
        self.toks = torch.zeros((B, k + 1), dtype=torch.int64, device=dev)  # [c, x_1 .. x_k] per row
        self.c = torch.zeros(B, dtype=torch.int64, device=dev)
        self.lens_t = torch.zeros(B, dtype=torch.int32, device=dev)
        self.lens_d = torch.zeros(B, dtype=torch.int32, device=dev)
        self.count = torch.zeros(B, dtype=torch.int64, device=dev)
        self.info = torch.zeros(4, dtype=torch.int64, device=dev)
        # pinned host slots the rounds' info is copied into (two rounds in
        # flight), with the event each copy completes
        self.info_host = [torch.zeros(4, dtype=torch.int64, pin_memory=True) for _ in range(2)]
        self.info_ev = [torch.cuda.Event() for _ in range(2)]
        self._slot = 0
        self.steps_i32 = torch.arange(k + 1, dtype=torch.int32, device=dev).view(k + 1, 1)
        self.out = None
        self.n_new = 0
        self.graph = None
        # the acceptance outputs (accept_len, out_ids, flags) of the most
        # recently ENQUEUED round: once captured, these are the graph's static
        # buffers, which every replay overwrites, so after run_rounds /
        # generate (a round is enqueued before the previous one's info is
        # read) they may already hold a later round than the info last
        # returned; step() enqueues one round and waits for it, so after
        # step() they are that round's
        self.last = None
        # attention prefix bound used by captured rounds
        self.bound_t = target.cap - (k + 2)
        self.bound_d = draft.cap - (k + 2)

    # ---- one round on the static buffers ---------------------------------
    def _fill_uniforms(self):
        if not self.greedy:
            torch.rand(self.u_all.shape, generator=self.gen, device=self.dev, out=self.u_all)

    def _round(self, Tmax_t: int, Tmax_d: int):
        B, k = self.B, self.k
        tok = self.c
        # the draft's positions lens_d[b] + i of all k+1 steps in one kernel
        lens_steps = self.lens_d.view(1, B) + self.steps_i32
        for i in range(k + 1):
            # the last step only writes the last draft token's cache rows
            h = self.d.forward(tok.view(B, 1), lens_steps[i], Tmax_d + i, out_dtype=self.d.act_dtype,
                               cache_only=i == k)
            if i == k:
                break
            self.d.logits(h, out=self.qbuf[:, i:i + 1])
            if self.greedy:
                self.xsT[i].copy_(self.hip.argmax(self.qbuf[:, i]).view(B))
            else:
                self.hip.sample(self.qbuf[:, i], self.u_draft[i], temperature=self.T, out=self.xsT[i],
                                lse_out=self.lse_dr[i], flags_out=self.fl_dr[i])
            tok = self.xsT[i]
        torch.cat([self.c.view(B, 1), self.xsT.t()], dim=1, out=self.toks)
        xs = self.toks[:, 1:]
        h = self.t.forward(self.toks, self.lens_t, Tmax_t, out_dtype=self.t.act_dtype)
        self.t.logits(h, out=self.pbuf)
        if self.greedy:
            _, _, alen, ids = self.hip.greedy_verify(self.pbuf, xs, rows_t=k + 1)
            self.last = dict(accept_len=alen, out_ids=ids, flags=None)
        else:
            res = self.hip.spec_accept(self.pbuf, self.qbuf, xs, self.u_acc, temperature=self.T,
                                       lse_d_in=self.lse_dr, flags_d_in=self.fl_dr)
            alen, ids = res["accept_len"], res["out_ids"]
            self.last = res
        # commit (one launch, no data-dependent shapes, so the round can be
        # captured): ids[b, :n_b + 1] appended to out[b, count_b ...], counts,
        # cache lengths and the next round's first token advanced, and the
        # host's loop summary in info
        P = ctypes.c_void_p
        _lib.check(self.hip._L.vnx_spec_commit(
            P(alen.data_ptr()), P(ids.data_ptr()), ids.stride(0), B, k, P(self.out.data_ptr()), self.out.stride(0),
            self.out.shape[1] - 1, P(self.count.data_ptr()), P(self.c.data_ptr()), P(self.lens_t.data_ptr()),
            P(self.lens_d.data_ptr()), P(self.info.data_ptr()),
            ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)), "spec_commit")

    # ---- driver ---------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompts: torch.Tensor, n_new: int) -> float:
        """Runs the prompts (B, T0) int64 on the device through both models,
        resets the round state and the output buffer for n_new tokens per
        sequence, and returns the prefill wall time (s).  Rounds then follow
        with step()."""
        B, T0 = prompts.shape
        if B != self.B:
            raise ValueError(f"batch {B} != {self.B}")
        if T0 < 1:
            raise ValueError("prompts need at least one token")
        k = self.k
        dev = self.dev
        if T0 - 1 + n_new + 2 * (k + 1) > min(self.t.cap, self.d.cap):
            raise ValueError("the caches cannot hold prompt + n_new tokens")
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        self.lens_t.zero_()
        self.lens_d.zero_()
        if T0 > 1:
            self.t.forward(prompts[:, :-1], self.lens_t, 0)
            self.d.forward(prompts[:, :-1], self.lens_d, 0)
        self.lens_t += T0 - 1
        self.lens_d += T0 - 1
        self.c.copy_(prompts[:, -1])
        self.count.zero_()
        if self.out is None or self.n_new != n_new:
            self.out = torch.full((B, n_new + k + 2), -1, dtype=torch.int64, device=dev)
            self.n_new = n_new
            self.graph = None
        else:
            self.out.fill_(-1)
        self._Tmax = (T0 - 1, T0 - 1)
        torch.cuda.synchronize(dev)
        return time.perf_counter() - t0

    def _set_uniforms(self, uniforms) -> None:
        """uniforms = (u_draft (k, B), u_acc (B, k+1)) float32 (host arrays or
        tensors): u_draft[i, b] draws draft token i+1 of sequence b from
        softmax(q_i / T); u_acc[b, :k] are its acceptance tests and
        u_acc[b, k] its residual / bonus draw."""
        ud, ua = uniforms
        ud = torch.as_tensor(ud, dtype=torch.float32)
        ua = torch.as_tensor(ua, dtype=torch.float32)
        if tuple(ud.shape) != tuple(self.u_draft.shape) or tuple(ua.shape) != tuple(self.u_acc.shape):
            raise ValueError(f"uniforms must be ({self.k}, {self.B}) and ({self.B}, {self.k + 1})")
        self.u_draft.copy_(ud)
        self.u_acc.copy_(ua)

    def _launch(self, uniforms=None) -> int:
        """Enqueues one round (a graph replay once captured) and the copy of
        its info into a pinned host slot; returns the slot."""
        if self.out is None:
            raise RuntimeError("call prefill() before step()")
        if uniforms is None:
            self._fill_uniforms()
        elif not self.greedy:
            self._set_uniforms(uniforms)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._round(*self._Tmax)
        slot = self._slot
        self._slot ^= 1
        self.info_host[slot].copy_(self.info, non_blocking=True)
        self.info_ev[slot].record(torch.cuda.current_stream(self.dev))
        return slot

    def _collect(self, slot: int) -> torch.Tensor:
        """Waits for the round whose info went to slot and returns that info
        (checking that the next round fits the caches)."""
        self.info_ev[slot].synchronize()
        info = self.info_host[slot].clone()
        Tmax_t, Tmax_d = int(info[1]), int(info[2])
        if Tmax_t + self.k + 2 > self.t.cap or Tmax_d + self.k + 2 > self.d.cap:
            if int(info[0]) < self.n_new:
                raise RuntimeError("KV cache capacity exhausted")
        self._Tmax = (Tmax_t, Tmax_d)
        return info

    def _fits_ahead(self) -> bool:
        """Whether a round may be enqueued before the previous round's info
        is read: graph replays only (eager rounds size their attention calls
        by it), and the caches must hold the round after next even if every
        draft of the round in flight is accepted."""
        if self.graph is None:
            return False
        Tt, Td = self._Tmax
        grow = 2 * (self.k + 1) + 1
        return Tt + grow <= self.t.cap and Td + grow <= self.d.cap

    @torch.no_grad()
    def step(self, uniforms=None) -> torch.Tensor:
        """One speculative round of every sequence (a graph replay once
        captured).  uniforms: None (drawn from the engine's generator) or
        (u_draft, u_acc) supplied by the caller (see _set_uniforms).  Returns
        info (4,) int64 on the host: min committed count, max target / draft
        cache length, accepted drafts summed over the batch."""
        return self._collect(self._launch(uniforms))

    @torch.no_grad()
    def run_rounds(self, n: int, uniforms=None) -> list:
        """n rounds back to back, each round enqueued before the previous
        one's info is read (while the caches allow it), so the GPU does not
        wait on the host between rounds.  Returns the n infos (see step())."""
        infos = []
        if n <= 0:
            return infos
        pending = self._launch(None if uniforms is None else uniforms(0))
        for r in range(1, n + 1):
            nxt = None
            if r < n and self._fits_ahead():
                nxt = self._launch(None if uniforms is None else uniforms(r))
            infos.append(self._collect(pending))
            if r < n and nxt is None:
                nxt = self._launch(None if uniforms is None else uniforms(r))
            pending = nxt
        return infos

    @torch.no_grad()
    def generate(self, prompts: torch.Tensor, n_new: int, phase_timing: bool = False, uniforms=None):
        """prompts (B, T0) int64 on the device.  Returns (tokens (B, n_new)
        int64 on the device, DecodeStats).  Prefill is timed separately from
        the decode rounds.  uniforms: None, or a callable round_index ->
        (u_draft, u_acc) giving each round's uniforms (see step()).
        A round is enqueued before the previous one's info is read whenever
        that round certainly is not the last (the slowest sequence still
        needs more than k + 1 tokens) and the caches allow it; the rounds
        and their uniforms are the same as with one round at a time."""
        B, k = self.B, self.k
        st = DecodeStats(prefill_s=self.prefill(prompts, n_new))
        if self.use_graph and self.graph is None:
            self._capture()
        t1 = time.perf_counter()
        low = 0                                    # min committed count known so far
        pending = self._launch(None if uniforms is None else uniforms(0))
        launched = 1
        while True:
            ta = time.perf_counter()
            nxt = None
            if low + (k + 1) < n_new and self._fits_ahead():
                nxt = self._launch(None if uniforms is None else uniforms(launched))
                launched += 1
            info = self._collect(pending)
            st.rounds += 1
            st.per_round_tokens.append(int(info[3]) + B)
            if phase_timing:
                st.draft_s += time.perf_counter() - ta
            low = int(info[0])
            if low >= n_new:
                break                              # nxt is None here: low + k + 1 < n_new was false
            if nxt is None:
                nxt = self._launch(None if uniforms is None else uniforms(launched))
                launched += 1
            pending = nxt
        torch.cuda.synchronize(self.dev)
        st.decode_s = time.perf_counter() - t1
        st.emitted = B * n_new
        st.accepted_drafts = sum(st.per_round_tokens) - B * st.rounds
        return self.out[:, :n_new].clone(), st

    def _capture(self):
        """Captures one round on a side stream.  Warm-up rounds on that stream
        first allocate every workspace and cached tensor; the caches and
        counters they touch are restored afterwards (the warm-up only writes
        cache rows past every lens[b], which later rounds overwrite)."""
        saved = [x.clone() for x in (self.c, self.lens_t, self.lens_d, self.count, self.out)]
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            for _ in range(2):
                self._fill_uniforms()
                self._round(self.bound_t, self.bound_d)
                for x, v in zip((self.c, self.lens_t, self.lens_d, self.count, self.out), saved):
                    x.copy_(v)
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self._round(self.bound_t, self.bound_d)
        torch.cuda.synchronize(self.dev)
        for x, v in zip((self.c, self.lens_t, self.lens_d, self.count, self.out), saved):
            x.copy_(v)
        self.graph = g
