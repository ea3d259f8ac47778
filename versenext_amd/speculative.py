"""SpeculativeDecoder: VerseNext's speculative-decode entry point on MI355X.

Keeps the reference class's constructor and method signatures
(packages/verse_nex/verse_nex/speculative.py:55-348):
  SpeculativeDecoder(dim, vocab_size, num_draft_heads=4, shared_embedding=None)
  .draft(hidden, last_position=None) -> (np.ndarray int64 (B,k), [k logits (B,V)])
  .verify(draft_tokens, main_model, context_tokens) -> (bool (B,k), int64 (B,k))
  .verify_then_commit(draft_tokens, main_model, context_tokens, max_redraft_rounds=1)
      -> (list[int], bool, np.ndarray (1, T_ctx + n))
  .draft_loss(draft_logits, target_tokens) -> scalar
with the same errors (ValueError for num_draft_heads < 1, non-2-D inputs,
batch mismatch, bad hidden rank).  One keyword is added, `device`
(default "rocm"): the argmax of the draft heads, the verify argmax and the
accept-prefix rule run in the gfx950 kernels (vnx_row_argmax,
vnx_greedy_verify); the draft heads' GEMM runs in rocBLAS.

Batched extensions (no reference counterpart; the reference verifies batch
row 0 only, speculative.py:262-268):
  .verify_batch(...)  greedy verify + commit for every row, optional bonus token;
  .accept(...)        stochastic acceptance with explicit uniforms (vnx_spec_accept).
"""
from __future__ import annotations

from typing import Callable, List, Optional, Tuple

import numpy as np
import torch

from .device import get_backend
from .hip_backend import _to_tensor


class DraftHead:
    """Linear(dim, vocab, bias=False) on the device: y = x @ W.T, W (vocab, dim)
    (packages/verse_torch/verse_torch/vnnn.py:394-430)."""

    def __init__(self, owner: "SpeculativeDecoder", weight: torch.Tensor):
        self._owner = owner
        self._weight = weight

    @property
    def weight(self) -> torch.Tensor:
        return self._weight

    @weight.setter
    def weight(self, w) -> None:
        rg = bool(getattr(w, "requires_grad", False))
        t = _to_tensor(w, self._owner.device, torch.float32).detach().clone()
        if tuple(t.shape) != (self._owner.vocab_size, self._owner.dim):
            raise ValueError(f"draft head weight must be ({self._owner.vocab_size}, {self._owner.dim})")
        self._weight = t.requires_grad_(rg)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return torch.nn.functional.linear(x, self._weight)


class SpeculativeDecoder:
    def __init__(self, dim: int, vocab_size: int, num_draft_heads: int = 4,
                 shared_embedding=None, device: str = "rocm", seed: Optional[int] = None):
        if num_draft_heads < 1:
            raise ValueError(f"num_draft_heads must be >= 1, got {num_draft_heads}")
        self.dim = int(dim)
        self.vocab_size = int(vocab_size)
        self.num_draft_heads = int(num_draft_heads)
        self.shared_embedding = shared_embedding
        self.backend = get_backend(device)
        self.device = self.backend.torch_device
        g = torch.Generator(device="cpu")
        if seed is not None:
            g.manual_seed(int(seed))
        bound = 1.0 / np.sqrt(self.dim)  # Kaiming-uniform bound of a Linear(dim, .) layer
        self.draft_heads: List[DraftHead] = []
        for _ in range(self.num_draft_heads):
            w = (torch.rand((self.vocab_size, self.dim), generator=g) * 2 - 1) * bound
            self.draft_heads.append(DraftHead(self, w.to(self.device).requires_grad_(True)))

    # ------------------------------------------------------------------
    def _hidden_last(self, hidden) -> torch.Tensor:
        h = _to_tensor(hidden, self.device, torch.float32)
        if h.dim() == 2:
            return h
        if h.dim() == 3:
            return h[:, -1, :]
        if h.dim() == 4:
            return h.reshape(h.shape[0], -1, h.shape[-1])[:, -1, :]
        raise ValueError(f"hidden has {h.dim()} dims; expected 2, 3 or 4")

    def draft(self, hidden, last_position: Optional[int] = None) -> Tuple[np.ndarray, List[torch.Tensor]]:
        """k head logits (B, V) and their argmax tokens (speculative.py:110-162)."""
        h = self._hidden_last(hidden)
        logits = [head(h) for head in self.draft_heads]  # (B, V) each
        stacked = torch.stack([lg.detach() for lg in logits], dim=1)  # (B, k, V)
        toks = self.backend.argmax(stacked)  # (B, k)
        return toks.cpu().numpy().astype(np.int64), logits

    # ------------------------------------------------------------------
    def _run_main(self, main_model: Callable, tokens: np.ndarray) -> torch.Tensor:
        full_t = torch.from_numpy(np.ascontiguousarray(tokens.astype(np.int64))).to(self.device)
        with torch.no_grad():
            out = main_model(full_t)
        logits = out[0] if isinstance(out, tuple) else out
        return _to_tensor(logits, self.device)

    def verify(self, draft_tokens, main_model: Callable, context_tokens) -> Tuple[np.ndarray, np.ndarray]:
        """accepted_mask (B,k) bool and main_pred (B,k) int64 (speculative.py:168-224)."""
        draft_tokens = np.asarray(draft_tokens)
        context_tokens = np.asarray(context_tokens)
        if draft_tokens.ndim != 2 or context_tokens.ndim != 2:
            raise ValueError("draft_tokens / context_tokens must be 2-D (B, k) / (B, T_ctx)")
        if draft_tokens.shape[0] != context_tokens.shape[0]:
            raise ValueError(f"batch mismatch: draft {draft_tokens.shape[0]} vs context {context_tokens.shape[0]}")
        B, k = draft_tokens.shape
        T_ctx = context_tokens.shape[1]
        logits = self._run_main(main_model, np.concatenate([context_tokens, draft_tokens], axis=1))
        window = logits[:, T_ctx - 1:T_ctx - 1 + k, :]
        acc, pred, _, _ = self.backend.greedy_verify(window, draft_tokens, rows_t=k)
        return acc.cpu().numpy(), pred.cpu().numpy().astype(np.int64)

    def verify_then_commit(self, draft_tokens, main_model: Callable, context_tokens,
                           max_redraft_rounds: int = 1) -> Tuple[List[int], bool, np.ndarray]:
        """Longest accepted prefix of batch row 0 plus the target's token at the
        first mismatch; no bonus token (speculative.py:230-310)."""
        draft_tokens = np.asarray(draft_tokens)
        context_tokens = np.asarray(context_tokens)
        d_b, c_b = draft_tokens[:1], context_tokens[:1]
        B, k = d_b.shape
        T_ctx = c_b.shape[1]
        logits = self._run_main(main_model, np.concatenate([c_b, d_b], axis=1))
        window = logits[:1, T_ctx - 1:T_ctx - 1 + k, :]
        _, _, alen, out = self.backend.greedy_verify(window, d_b, rows_t=k)
        n = int(alen[0].item())
        all_accepted = n == k
        emitted = n if all_accepted else n + 1
        accepted_tokens = [int(v) for v in out[0, :emitted].cpu().tolist()]
        new_ctx = np.concatenate([c_b, np.asarray(accepted_tokens, dtype=np.int64)[None, :]], axis=1)
        if not all_accepted and max_redraft_rounds > 0:
            full_t = torch.from_numpy(new_ctx.astype(np.int64)).to(self.device)
            with torch.no_grad():
                out_m = main_model(full_t)
            if isinstance(out_m, tuple):
                hid = out_m[1] if len(out_m) > 1 else out_m[0]
            else:
                hid = out_m
            self.draft(hid)
        return accepted_tokens, all_accepted, new_ctx

    # ------------------------------------------------------------------
    def verify_batch(self, draft_tokens, main_model: Callable, context_tokens, bonus: bool = True):
        """Greedy verify + commit for every batch row. Returns (accept_len (B,) int32,
        out_ids (B, k+1) int64, -1 padded) as device tensors."""
        draft_tokens = np.asarray(draft_tokens)
        context_tokens = np.asarray(context_tokens)
        if draft_tokens.ndim != 2 or context_tokens.ndim != 2:
            raise ValueError("draft_tokens / context_tokens must be 2-D")
        if draft_tokens.shape[0] != context_tokens.shape[0]:
            raise ValueError("batch mismatch")
        B, k = draft_tokens.shape
        T_ctx = context_tokens.shape[1]
        logits = self._run_main(main_model, np.concatenate([context_tokens, draft_tokens], axis=1))
        rows = k + 1 if bonus else k
        window = logits[:, T_ctx - 1:T_ctx - 1 + rows, :]
        _, _, alen, out = self.backend.greedy_verify(window, draft_tokens, rows_t=rows)
        return alen, out

    def accept(self, target_logits, draft_logits, draft_ids, uniforms, temperature: float = 1.0,
               thr_t=None, thr_d=None):
        """Stochastic acceptance (Leviathan et al. 2023, Alg. 1) on device; see
        HipBackend.spec_accept."""
        return self.backend.spec_accept(target_logits, draft_logits, draft_ids, uniforms,
                                        temperature=temperature, thr_t=thr_t, thr_d=thr_d)

    # ------------------------------------------------------------------
    def draft_loss(self, draft_logits: List[torch.Tensor], target_tokens) -> torch.Tensor:
        """Mean over heads of the cross-entropy of each head (speculative.py:316-348)."""
        target_tokens = np.asarray(target_tokens)
        if target_tokens.shape[1] != len(draft_logits):
            raise ValueError(f"target_tokens has {target_tokens.shape[1]} columns, "
                             f"draft_logits has {len(draft_logits)} heads")
        tgt = torch.from_numpy(target_tokens.astype(np.int64)).to(self.device)
        total = torch.zeros((), dtype=torch.float32, device=self.device)
        for i, lg in enumerate(draft_logits):
            total = total + torch.nn.functional.cross_entropy(lg.float(), tgt[:, i])
        return total * (1.0 / len(draft_logits))


__all__ = ["SpeculativeDecoder", "DraftHead"]
