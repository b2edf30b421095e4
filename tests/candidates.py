"""Which finalisation path the sampling kernels take for a row (test helper).

The library's streaming pass keeps, per 2048-element chunk, the elements
whose chunk-relative exponent RN32(x c - mc_j) reaches -L ("candidates"),
L chosen from the chunk's data: the largest level in [0, 31] at which at most
cap of the lanes' 16-byte vectors hold a candidate (by their vector maxima),
then lowered while more than cap elements qualify (none kept when even L = 0
leaves more than cap: the chunk overflows). The finaliser selects the top-p
cutoff among the candidates and takes one of these paths:

  fast        the cutoff exceeds every chunk's bound on the p of its
              non-candidates (p is monotone in the logit, so the bound is the
              p at the level's threshold, rounded up);
  refill      it does not: the chunks whose bound reaches it are re-read and
              their {p >= cutoff} replaces their candidates (fits in 2048
              entries), then the cutoff is selected again;
  slow_list   the candidates hold less than top_p, or the refill overflows:
              the whole row is selected by passes over it, and its support
              (<= 2048 elements) is kept in the entries;
  slow_dense  as slow_list with a larger support: the draws pass over the row.

The paths must give identical results; the oracle computes the result
directly. This restates the candidate rule for rows without a penalty (x in
binary32, T = 1 unless given), so that tests can build rows taking each path.
"""

from __future__ import annotations

import numpy as np

from oracle import native
from oracle import numerics as nm
from oracle import sampling as osmp

CHUNK = 2048
LANES = 64
ROW_CAP = 2048
MAX_LEVEL = 31


def chunk_cap(nch: int) -> int:
    """Candidate slots per chunk for a row of nch chunks (nch * cap <= 2048)."""
    return 64 if nch <= 32 else (32 if nch <= 64 else 16)


def _chunk_candidates(xs: np.ndarray, c: np.float32, mc: np.float32, cap: int, epv: int):
    """(level or -1 on overflow, candidate mask) of one chunk."""
    n = len(xs)
    nvc = CHUNK // (LANES * epv)
    pad = np.full(CHUNK, -np.inf, dtype=np.float32)
    pad[:n] = xs
    vec = pad.reshape(nvc * LANES, epv)          # vector v = u * 64 + t
    valid_vec = np.arange(nvc * LANES) * epv < n
    vm = np.where(valid_vec, vec.max(axis=1), -np.inf).astype(np.float32)
    tv = nm.fma32(vm, c, -mc)
    tx = nm.fma32(xs, c, -mc)

    def nv(level):
        return int((tv >= np.float32(-level)).sum())

    lo, hi = 0, MAX_LEVEL
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if nv(mid) <= cap:
            lo = mid
        else:
            hi = mid - 1
    for level in range(lo, -1, -1):
        mask = tx >= np.float32(-level)
        if mask.sum() <= cap:
            return level, mask
    return -1, np.zeros(n, dtype=bool)


def row_path(x: np.ndarray, top_p: float, temperature: float = 1.0, epv: int = 4) -> str:
    pr = osmp.process_logits(np.asarray(x, dtype=np.float32), temperature, epv=epv)
    soft = osmp.softmax_row(pr)
    if top_p >= 1.0:
        return "unfiltered"
    v = len(pr.x)
    nch = -(-v // CHUNK)
    cap = chunk_cap(nch)
    cand = np.zeros(v, dtype=bool)
    bounds = []
    for j in range(nch):
        xs = pr.x[j * CHUNK:(j + 1) * CHUNK]
        mc = soft.mc_chunks[j]
        level, mask = _chunk_candidates(xs, pr.c, mc, cap, epv)
        cand[j * CHUNK:(j + 1) * CHUNK] = mask
        if not mc > -np.inf:
            bounds.append(0.0)
        elif level < 0:
            bounds.append(np.inf)
        else:
            tb = (float(mc) - level) * (pr.cd / float(pr.c)) - float(soft.mcmax)
            tf = np.nextafter(np.float32(tb), np.float32(np.inf))
            bounds.append(float(native.exp2p(np.float32([tf]))[0] / soft.s))
    p = soft.p
    thr = osmp.threshold_fx(top_p)
    pc = np.where(cand, p, np.float32(0.0))
    support = lambda c: int((p >= c).sum())  # noqa: E731
    if int(nm.fx46(pc).sum(dtype=np.uint64)) < thr:
        cut, _ = osmp.top_p_cutoff(p, top_p)
        return "slow_list" if support(cut) <= ROW_CAP else "slow_dense"
    cut, _ = osmp.top_p_cutoff(pc, top_p)
    if cut > max(bounds):
        return "fast"
    entries = 0
    for j in range(nch):
        seg = slice(j * CHUNK, (j + 1) * CHUNK)
        entries += int((p[seg] >= cut).sum()) if bounds[j] >= cut else int(cand[seg].sum())
    if entries <= ROW_CAP:
        return "refill"
    true_cut, _ = osmp.top_p_cutoff(p, top_p)
    return "slow_list" if support(true_cut) <= ROW_CAP else "slow_dense"


def path_rows(seed: int = 0) -> dict:
    """Constructed float32 rows (T = 1) for each path: {name: (row, top_p)}.

    refill (V = 16384, top_p 0.5): chunk 0 holds 50 tokens at 6.0, chunk 1
      100 tokens tied at 5.0 (more than its 64 slots: it overflows and keeps
      no candidates), chunks 2..7 hold 60 tokens at 4.5 each. The candidates
      reach 0.5 inside the 4.5 tokens, chunk 1 is re-read, its ties join, and
      the cutoff moves up to them.
    slow_list (V = 8192, top_p 0.9): 1500 tokens tied at 5.0 spread over
      every chunk (375 each: every chunk overflows), the rest far below: the
      candidates hold nothing; the support of 1500 fits the entries.
    slow_dense: as slow_list with 3000 ties.
    fast (V = 8192, top_p 0.9): a Gaussian row with a few dominant tokens.
    """
    rng = np.random.default_rng(seed)
    refill = (rng.standard_normal(16384) * 0.5 - 8.0).astype(np.float32)
    refill[rng.choice(CHUNK, 50, replace=False)] = 6.0
    refill[CHUNK + rng.choice(CHUNK, 100, replace=False)] = 5.0
    for j in range(2, 8):
        refill[j * CHUNK + rng.choice(CHUNK, 60, replace=False)] = 4.5
    slow_list = np.full(8192, -30.0, dtype=np.float32)
    slow_list[np.linspace(0, 8191, 1500).astype(np.int64)] = 5.0
    slow_dense = np.full(8192, -30.0, dtype=np.float32)
    slow_dense[np.linspace(0, 8191, 3000).astype(np.int64)] = 5.0
    fast = (rng.standard_normal(8192) * 3).astype(np.float32)
    fast[rng.choice(8192, 30, replace=False)] = 14.0
    return {"refill": (refill, 0.5), "slow_list": (slow_list, 0.9), "slow_dense": (slow_dense, 0.9),
            "fast": (fast, 0.9)}
