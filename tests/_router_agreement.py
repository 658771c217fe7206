"""Row-by-row agreement of a top-k router with transformers' router.

Test helper.  Two routers that compute the same bf16 logits pick the same
expert set, except where the k-th largest logit is tied: the build keeps
the lower expert id, torch.topk leaves the choice unspecified.  Where the
logits differ (a different fp32 summation order can move a logit by one
bf16 ulp), the sets may differ only through experts whose logit sits within
one ulp of the k-th logit.  ``classify`` asserts exactly that and returns
the counts reported in the design notes.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Agreement:
    rows: int = 0
    exact_logit_rows: int = 0      # logits bitwise equal to transformers'
    same_set_rows: int = 0         # same selected experts (as a set)
    tie_rows: int = 0              # set differs: tie at the k-th logit, equal logits
    flip_rows: int = 0             # logits differ by one ulp somewhere
    flip_set_rows: int = 0         # ... and the set differs through such a flip

    @property
    def agreement(self) -> float:
        return self.same_set_rows / self.rows if self.rows else 1.0


def _ordered(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> integers in the order of the values they encode
    (adjacent values differ by one)."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, 0x8000 - b, b)


def classify(logits: np.ndarray, index: np.ndarray, hf_logits: np.ndarray,
             hf_index: np.ndarray, top_k: int) -> Agreement:
    """``logits``/``hf_logits``: bf16 bits [T, E]; ``index``/``hf_index``:
    int [T, K].  Raises AssertionError on any difference that is neither a
    tie at the k-th logit nor a one-ulp logit flip."""
    out = Agreement()
    ours_o, hf_o = _ordered(logits), _ordered(hf_logits)
    for t in range(logits.shape[0]):
        out.rows += 1
        mine, theirs = set(index[t].tolist()), set(hf_index[t].tolist())
        same = mine == theirs
        out.same_set_rows += same
        dist = np.abs(ours_o[t] - hf_o[t])
        assert dist.max() <= 1, f"row {t}: logits differ by {dist.max()} ulps"
        kth = np.sort(ours_o[t])[::-1][top_k - 1]
        if dist.max() == 0:
            out.exact_logit_rows += 1
            if not same:
                out.tie_rows += 1
                for e in mine ^ theirs:
                    assert ours_o[t, e] == kth, f"row {t}: expert {e} is not tied at the k-th logit"
        else:
            out.flip_rows += 1
            if not same:
                out.flip_set_rows += 1
                for e in mine ^ theirs:
                    assert abs(int(ours_o[t, e]) - int(kth)) <= 1, \
                        f"row {t}: expert {e} differs by more than a boundary flip"
    return out
