"""Routing against the reference's literal ops: torch.sigmoid, + bias, torch.topk
(abacus/moe/router.py:45-48), in the activation dtype.

The kernel's routing is bit-exact against the oracle's canonical form (correctly rounded
sigmoid, ties to the lower expert index). torch's own ops can only disagree with that form
in two ways, and a token is exempt from the exact-set comparison only when one of them can
reach its top-k boundary:
  (a) a tie: torch's k-th and (k+1)-th selection values are exactly equal, so torch.topk's
      choice among the tied experts is implementation-defined;
  (b) a sigmoid difference at the boundary: each expert's selection value lies in the
      interval [lo, hi] spanned by its values under the two sigmoids (a single point where
      they agree), and the token is exempt when some expert in torch's top-k has lo at or
      below the hi of some expert outside it -- only then can the kernel's values order the
      two the other way.
Every other token must pick exactly torch.topk's set. On exempt tokens the kernel's set
must still be a valid top-k: for a tie, every pick's torch value at least every
non-pick's; for (b), every pick's hi at least every non-pick's lo.
"""

from __future__ import annotations

import dataclasses

import torch


@dataclasses.dataclass
class TopkCheck:
    tokens: int
    ties: int              # exempt by (a)
    sigmoid_exempt: int    # exempt by (b) and not by (a)
    set_mismatches: int    # non-exempt tokens whose set differs from torch.topk's
    invalid_exempt: int    # exempt tokens whose set is not a valid top-k under torch's values

    @property
    def exempt(self) -> int:
        return self.ties + self.sigmoid_exempt

    def summary(self) -> str:
        return (f"tokens {self.tokens}: ties {self.ties}, sigmoid-boundary {self.sigmoid_exempt} "
                f"(exempt {100.0 * self.exempt / max(self.tokens, 1):.2f}%), "
                f"set mismatches {self.set_mismatches}, invalid exempt sets {self.invalid_exempt}")


def check_against_torch_topk(logits: torch.Tensor, bias_E: torch.Tensor, picked: torch.Tensor,
                             scores_cr: torch.Tensor) -> TopkCheck:
    """Compare picked (T,K) expert sets with torch.sigmoid + bias + torch.topk on the CPU.

    logits (T,E) and bias_E (E,) in the activation dtype; scores_cr (T,E) the correctly
    rounded sigmoid in that dtype (the kernel's).
    """
    logits = logits.cpu()
    bias_E = bias_E.cpu()
    picked = picked.cpu().long()
    T, E = logits.shape
    K = picked.shape[-1]
    sel_t = (torch.sigmoid(logits) + bias_E).float()
    sel_k = (scores_cr.cpu() + bias_E).float()
    torch_idx = torch.topk(torch.sigmoid(logits) + bias_E, K, dim=-1).indices
    same = (torch.sort(picked, -1).values == torch.sort(torch_idx, -1).values).all(-1)
    if K >= E:
        return TopkCheck(T, 0, 0, int((~same).sum()), 0)

    v = torch.sort(sel_t, dim=-1, descending=True).values
    kth, k1 = v[:, K - 1:K], v[:, K:K + 1]
    tie = (kth == k1).squeeze(-1)
    lo = torch.minimum(sel_t, sel_k)
    hi = torch.maximum(sel_t, sel_k)
    inf = torch.tensor(float("inf"))
    tmask = torch.zeros(T, E, dtype=torch.bool)
    tmask.scatter_(1, torch_idx, True)
    cross = torch.where(tmask, lo, inf).amin(-1) <= torch.where(tmask, -inf, hi).amax(-1)
    sig = cross & ~tie
    exempt = tie | sig

    mask = torch.zeros(T, E, dtype=torch.bool)
    mask.scatter_(1, picked, True)
    valid_tie = torch.where(mask, sel_t, inf).amin(-1) >= torch.where(mask, -inf, sel_t).amax(-1)
    valid_sig = torch.where(mask, hi, inf).amin(-1) >= torch.where(mask, -inf, lo).amax(-1)
    valid = torch.where(tie, valid_tie, valid_sig)
    return TopkCheck(T, int(tie.sum()), int(sig.sum()), int((~same & ~exempt).sum()),
                     int((exempt & ~valid).sum()))
