"""Which finalisation path the sampling kernels take for a row (test helper).

The library finds a row's top-p cutoff among each chunk's largest entries (its
"candidates") and falls back to exact work only when that cannot be shown to
be the row's cutoff. This helper restates the candidate rule of the chunk
kernel on the CPU, from the declared arithmetic in oracle/, so that tests can
build rows that take each path:

  fast    the candidates' cutoff exceeds the worst-case bound on every p
          outside the candidates (kCandScale * 2^-K_j * g_j per chunk);
  repair  it does not, but re-reading the chunks whose bound reaches it shows
          every non-candidate p below it (the candidates' cutoff stands);
  rebuild some non-candidate reaches it, and in every chunk whose bound
          reaches it {p >= the candidates' cutoff} fits the chunk's slots: those
          chunks' candidates are replaced by that set and selected again;
  slow    otherwise, or when the candidates hold less than top_p: the whole
          row is selected exactly.

The four paths must give identical results; the oracle computes the result
directly, without candidates.
"""

from __future__ import annotations

import numpy as np

from oracle import numerics as nm
from oracle import sampling as osmp

CHUNK = 2048
CAND_SCALE = np.float32(1.41422)
BINS = 16


def chunk_caps(nch: int) -> int:
    """Candidate slots per chunk for a row of nch chunks (2048 per row)."""
    return 64 if nch <= 32 else (32 if nch <= 64 else 16)


def row_path(x: np.ndarray, temperature: float, top_p: float, epv: int = 4) -> str:
    pr = osmp.process_logits(np.asarray(x, dtype=np.float32), temperature, epv=epv)
    soft = osmp.softmax_row(pr.x, pr.c, epv)
    nch = len(soft.mc_chunks)
    cap = chunk_caps(nch)
    cand = np.zeros(len(pr.x), dtype=bool)
    ths, bounds = [], []
    for j in range(nch):
        xs = pr.x[j * CHUNK:(j + 1) * CHUNK]
        t = nm.fma32(xs, np.float32(pr.c), -np.float32(soft.mc_chunks[j]))
        e, k = nm.exp2q_k(t)
        cum = np.cumsum(np.bincount(np.clip(-k, 0, BINS - 1), minlength=BINS))
        K = 0
        while K < BINS and cum[K] <= cap:
            K += 1
        if K >= BINS:
            th = np.float32(np.ldexp(np.float32(1.0), -149))  # every e > 0
            bound = np.float32(0.0)
        elif K == 0:
            th = np.float32(np.inf)
            bound = np.float32(np.inf)
        else:
            th = np.float32(np.ldexp(CAND_SCALE, -K))
            bound = np.float32(th * soft.g_chunks[j])
        cand[j * CHUNK:(j + 1) * CHUNK] = e >= th
        ths.append(th)
        bounds.append(bound)
    p = soft.p
    thr = nm.fx46(np.float32(top_p))
    pc = np.where(cand, p, np.float32(0.0))
    if int(nm.fx46(pc).sum()) < int(thr):
        return "slow"
    cut, _ = osmp.top_p_cutoff(pc, top_p)
    if cut > max(bounds):
        return "fast"
    outside = p[~cand]
    if not (outside >= cut).any():
        return "repair"
    for j in range(nch):
        if bounds[j] >= cut and int((p[j * CHUNK:(j + 1) * CHUNK] >= cut).sum()) > cap:
            return "slow"
    return "rebuild"


def repair_rows(vocab: int = 4096) -> dict[str, np.ndarray]:
    """Rows of two chunks built to take the repair, rebuild and slow paths.

    repair / slow: chunk 1 holds 60 entries at its max (exponent bin 0) and
    10 just below (bin 1), so its K is 1 and only the 60 are candidates, with
    a worst-case bound of 0.7071 g on the rest. Chunk 0 (same max) holds one
    entry at the max and five at 2^-0.6, which set the cutoff at 0.66 g for
    top_p 0.9, below that bound. The ten bin-1 entries sit at 2^-1 (repair:
    they stay below the cutoff) or at 2^-0.52 (slow: they reach it, and chunk
    1's {p >= cutoff} is 70 entries, more than its 64 slots).

    rebuild: chunk 0 holds 40 entries at the max and 20 at 2^-0.6; chunk 1
    holds 50 at the max, 10 at 2^-0.52 and 5 at 2^-0.99 (15 in bin 1, so K is
    1 and its 50 max entries are its candidates). The candidates' cutoff is
    0.66 g, the ten at 2^-0.52 reach it, and chunk 1's {p >= cutoff} is 60.
    """
    ln2 = float(np.log(2.0))
    rows = {}
    for name, depth in (("repair", 1.0), ("slow", 0.52)):
        x = np.full(vocab, -30.0, dtype=np.float32)
        x[0] = 10.0
        x[100:105] = 10.0 - 0.6 * ln2
        x[CHUNK:CHUNK + 60] = 10.0
        x[CHUNK + 500:CHUNK + 510] = 10.0 - depth * ln2
        rows[name] = x
    x = np.full(vocab, -30.0, dtype=np.float32)
    x[0:40] = 10.0
    x[100:120] = 10.0 - 0.6 * ln2
    x[CHUNK:CHUNK + 50] = 10.0
    x[CHUNK + 500:CHUNK + 510] = 10.0 - 0.52 * ln2
    x[CHUNK + 700:CHUNK + 705] = 10.0 - 0.99 * ln2
    rows["rebuild"] = x
    return rows
