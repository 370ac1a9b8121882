"""Top-k set comparison with an explicit near-tie rule (shared by the indexer tests).

The reference's scores come from an fp32 einsum whose summation order is unspecified, and
torch.topk leaves tie order unspecified, so the reference itself only fixes the selected *set* up
to scores that agree within fp32 rounding.  A GPU index may differ from the oracle's exact-math
top-k only if its oracle score lies within `tol` of the oracle's k-th score (both directions).
"""
from __future__ import annotations

import numpy as np


def score_error_bound(q: np.ndarray, w_act: np.ndarray, keys: np.ndarray, extra_rel: float = 0.0) -> np.ndarray:
    """Per-(b, j) bound on |fp32 score - exact score|: 4*IC*2^-24 * sum_h |w_h| sum_c |q_hc k_jc| (+ extra)."""
    IC = q.shape[-1]
    mag = np.einsum("bhc,bsc->bhs", np.abs(q).astype(np.float64), np.abs(keys).astype(np.float64))
    mag = (mag * np.abs(w_act.astype(np.float64))[..., None]).sum(1)
    return mag * (4 * IC * 2.0 ** -24 + extra_rel)


def assert_topk_matches(gpu_idx: np.ndarray, scores: np.ndarray, k: int, tol: np.ndarray,
                        valid: np.ndarray | None = None) -> int:
    """Returns the number of near-tie substitutions accepted."""
    B, S = scores.shape
    subs = 0
    for b in range(B):
        nv = S if valid is None else int(min(S, max(0, valid[b])))
        kk = min(k, nv)
        got = gpu_idx[b]
        assert np.all(got[kk:] == -1), f"row {b}: expected -1 padding after {kk}"
        g = got[:kk]
        assert len(set(g.tolist())) == kk, f"row {b}: duplicate indices"
        assert np.all((g >= 0) & (g < nv)), f"row {b}: index out of range"
        if kk == 0:
            continue
        order = np.lexsort((np.arange(nv), -scores[b, :nv]))
        ref = order[:kk]
        kth = scores[b, ref[-1]]
        missing = set(ref.tolist()) - set(g.tolist())
        extra = set(g.tolist()) - set(ref.tolist())
        for j in list(missing) + list(extra):
            assert abs(scores[b, j] - kth) <= 2 * tol[b, j] + 2 * tol[b, ref[-1]], (
                f"row {b}: index {j} (score {scores[b, j]!r}) differs from the k-th score {kth!r} "
                f"by more than the fp32 bound")
        subs += len(extra)
        # returned order is descending in score (up to the same bound)
        s = scores[b, g]
        assert np.all(s[:-1] >= s[1:] - 2 * (tol[b, g[:-1]] + tol[b, g[1:]])), f"row {b}: not sorted by score"
    return subs
