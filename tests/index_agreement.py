"""Expert selection under the reference's own router arithmetic, compared with the
q-semantics router that the GPU kernels and the oracle share.

Reference arithmetic (src/hunyuan_moe_full.cpp):
  * logits: one sequential fp32 accumulator per (token, expert), products rounded
    before they are added (:414-423; g++ does not contract on x86-64 by default);
  * softmax: max-subtract, expf, sum, divide (:41-50);
  * top-k on the rounded probabilities, strict '<' so an equal later value stays
    behind (:56-82);
  * for the 32-layer stack, rms_norm_f32 with a sequential sum of squares
    (src/rms_norm.cpp:9-33) before the router.
q semantics (this build): logits in a 64-lane blocked fmaf order, RMSNorm in the same
blocked order, selection on the logits, ties to the lower index.

Both are exact restatements (the reference half is bit-exact against the reference's
own compiled source), so every place where they select differently is rounding.  This
module measures that on given inputs and checks it against a bound:

  With A_e = sum_h |x_h w_eh| and u = 2^-24, the sequential order is within
  gamma_H A_e of the exact dot, the blocked order (H/64 fmaf steps per lane, then a
  6-level tree) within gamma_(H/64+6) A_e.  A unit-weight RMSNorm computed two ways
  scales a row by factors within rho_seq + rho_blk of each other, rho <= (n/2 + 3) u
  for a sum of n terms.  So |l_ref(e) - l_q(e)| <= eps_e = c u A_e with
      c = 1.05 (H + H/64 + 6 + [H/2 + 3 + (H/64 + 6)/2 + 3 with the norm] + 2).
  If the two pick different experts i (q only) and j (reference only) for a token,
  then l_q(i) >= l_q(j) and l_ref(j) >= l_ref(i) up to the probability rounding, so
      0 <= l_q(i) - l_q(j) <= eps_i + eps_j + pi_ij,
  where pi_ij = 2u (6 + |l_i - m| + |l_j - m|) covers expf's argument rounding, two
  expf results within an ulp, and the division (m = the row's largest logit).  The
  same bound holds for two experts the methods order differently.

compare() asserts the elementwise bound for every (token, expert) and the pair bound
for every disagreement, and returns the counts (set and order differences, near ties,
probability ties, the worst disagreement against its bound).
"""
import concurrent.futures as cf
import os

import numpy as np

import hy_oracle as O

U = 2.0 ** -24
THREADS = min(16, os.cpu_count() or 1)


def _rows(T, n):
    step = max(1, -(-T // n))
    return [(lo, min(T, lo + step)) for lo in range(0, T, step)]


def _par(fn, T):
    with cf.ThreadPoolExecutor(THREADS) as ex:   # ctypes drops the GIL during each call
        list(ex.map(lambda r: fn(*r), _rows(T, THREADS)))


def logits_seq(x, wr):
    """The reference's router logits (src/hunyuan_moe_full.cpp:414-423)."""
    T, H = x.shape
    E = wr.shape[0]
    out = np.empty((T, E), np.float32)
    _par(lambda lo, hi: O.lib().hyo_router_logits_seq(O.fp(x[lo:hi]), O.fp(wr), hi - lo, H, E, O.fp(out[lo:hi])), T)
    return out


def logits_blocked(x, wr):
    """The q-semantics router logits (the GPU's order)."""
    T, H = x.shape
    E = wr.shape[0]
    out = np.empty((T, E), np.float32)
    _par(lambda lo, hi: O.lib().hyo_router_logits_blocked(O.fp(x[lo:hi]), O.fp(wr), hi - lo, H, E,
                                                          O.fp(out[lo:hi])), T)
    return out


def rms_norm_seq(x, eps=1e-5):
    """The reference's rms_norm_f32 with a unit weight (src/rms_norm.cpp:9-33)."""
    T, H = x.shape
    out = np.empty_like(x)
    ones = np.ones(H, np.float32)
    _par(lambda lo, hi: O.lib().hyo_rms_norm_f32(O.fp(x[lo:hi]), O.fp(ones), O.fp(out[lo:hi]), hi - lo, H,
                                                 np.float32(eps)), T)
    return out


def rms_norm_blocked(x, eps=1e-5):
    T, H = x.shape
    out = np.empty_like(x)
    _par(lambda lo, hi: O.lib().hyo_rms_norm_blocked_rows(O.fp(x[lo:hi]), None, O.fp(out[lo:hi]), hi - lo, H,
                                                          np.float32(eps)), T)
    return out


def ref_probs(lg):
    """softmax_f32 of every row (src/hunyuan_moe_full.cpp:41-50)."""
    p = np.array(lg, dtype=np.float32, copy=True)
    T, E = p.shape
    _par(lambda lo, hi: [O.lib().hyo_softmax_f32(O.fp(p[t]), E) for t in range(lo, hi)], T)
    return p


def bound_coeff(H, with_norm):
    c = H + H / 64 + 6 + 2
    if with_norm:
        c += H / 2 + 3 + (H / 64 + 6) / 2 + 3
    return 1.05 * c


def compare(x_ref, x_q, wr, K, with_norm=False):
    """Selections of the reference arithmetic (router input x_ref) and of the q semantics
    (router input x_q) for every token; asserts the rounding bounds and returns counts."""
    x_ref, x_q, wr = O.f32(x_ref), O.f32(x_q), O.f32(wr)
    T, H = x_q.shape
    E = wr.shape[0]
    l_r = logits_seq(x_ref, wr)
    l_q = logits_blocked(x_q, wr)
    w_r = np.empty((T, K), np.float32)
    i_r = np.empty((T, K), np.int32)
    O.lib().hyo_topkgating_easy(O.fp(l_r), T, E, K, O.fp(w_r), O.ip(i_r))
    _, i_q = O.route_topk(l_q, K)

    A = np.abs(x_q.astype(np.float64)) @ np.abs(wr.astype(np.float64)).T           # [T, E]
    eps = bound_coeff(H, with_norm) * U * A
    dl = np.abs(l_r.astype(np.float64) - l_q.astype(np.float64))
    assert (dl <= eps).all(), f"logit difference beyond the rounding bound: max ratio {(dl / eps).max():.3f}"
    m_r = l_r.max(axis=1).astype(np.float64)

    def slack(t, i, j):
        return eps[t, i] + eps[t, j] + 2 * U * (6 + abs(l_r[t, i] - m_r[t]) + abs(l_r[t, j] - m_r[t]))

    set_diff, order_diff, worst = [], [], 0.0
    for t in np.flatnonzero((np.sort(i_r, axis=1) != np.sort(i_q, axis=1)).any(axis=1)):
        only_q = np.setdiff1d(i_q[t], i_r[t])
        only_r = np.setdiff1d(i_r[t], i_q[t])
        for i in only_q:
            for j in only_r:
                gap = float(l_q[t, i]) - float(l_q[t, j])
                b = slack(t, i, j)
                assert -b <= gap <= b, f"token {t}: experts {i}/{j} differ by {gap:.3e} > bound {b:.3e}"
                worst = max(worst, abs(gap) / b)
        set_diff.append(int(t))
    same_set = np.flatnonzero((np.sort(i_r, axis=1) == np.sort(i_q, axis=1)).all(axis=1))
    for t in same_set[(i_r[same_set] != i_q[same_set]).any(axis=1)]:
        pos_q = {int(e): k for k, e in enumerate(i_q[t])}
        for a in range(K):
            for b_ in range(a + 1, K):
                ea, eb = int(i_r[t, a]), int(i_r[t, b_])
                if pos_q[ea] > pos_q[eb]:       # ordered differently
                    gap = float(l_q[t, ea]) - float(l_q[t, eb])
                    b = slack(t, ea, eb)
                    assert abs(gap) <= b, f"token {t}: order of {ea}/{eb} differs by {gap:.3e} > bound {b:.3e}"
                    worst = max(worst, abs(gap) / b)
        order_diff.append(int(t))

    # probability ties the reference resolves by index where the logits differ
    p = ref_probs(l_r)
    sel_p = np.take_along_axis(p, i_r, axis=1)
    sel_l = np.take_along_axis(l_r, i_r, axis=1)
    tie_sel = 0
    for t in range(T):
        _, inv, cnt = np.unique(sel_p[t], return_inverse=True, return_counts=True)
        for g in np.flatnonzero(cnt > 1):
            if np.unique(sel_l[t][inv == g]).size > 1:
                tie_sel += 1
                break
    # 8th/9th boundary under the q order: near ties (gap within the bound) are reported
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -l_q.astype(np.float64)), axis=1)
    e8, e9 = order[:, K - 1], order[:, K]
    tt = np.arange(T)
    gap89 = l_q[tt, e8].astype(np.float64) - l_q[tt, e9]
    b89 = eps[tt, e8] + eps[tt, e9] + 2 * U * (6 + np.abs(l_r[tt, e8] - m_r) + np.abs(l_r[tt, e9] - m_r))
    near = np.flatnonzero(gap89 <= b89)
    # the same boundary at a realistic scale: 64 u (A_8 + A_9), a few times the largest
    # difference the two orders show in practice (random-walk rounding, ~sqrt(H) u A)
    near64 = np.flatnonzero(gap89 <= 64 * U * (A[tt, e8] + A[tt, e9]))
    p_boundary_tie = int(np.sum((p[tt, e8] == p[tt, e9]) & (l_r[tt, e8] != l_r[tt, e9])))
    return {
        "tokens": T,
        "set_differs": len(set_diff),
        "order_differs": len(order_diff),
        "set_differs_tokens": set_diff[:20],
        "selected_prob_ties_with_distinct_logits": tie_sel,
        "boundary_prob_ties_with_distinct_logits": p_boundary_tie,
        "near_ties_8_9": int(near.size),
        "near_tie_tokens": [int(t) for t in near[:20]],
        "near_ties_8_9_64uA": int(near64.size),
        "near_tie_64uA_tokens": [int(t) for t in near64[:20]],
        "min_gap_8_9": float(gap89.min()),
        "max_logit_diff_over_uA": float((dl / (U * A)).max()),
        "bound_coeff": bound_coeff(H, with_norm),
        "worst_disagreement_over_bound": worst,
    }
