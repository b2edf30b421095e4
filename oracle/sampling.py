"""Sampling-path oracle on the declared arithmetic (numpy; test infrastructure).

Every function restates one reference function; the docstring cites it. Rows
are processed independently. "p" is a softmax probability, "P" a filtered and
renormalised probability; masses are exact 2^-46 fixed-point integers (see
oracle.numerics). Parity status per function:

- softmax_row, top_p_cutoff, filter_row, categorical_pick: pinned against
  torch-CPU restatements (oracle.torch_ref) on seeded inputs, brute force on
  tiny vocabularies and closed-form special cases (tests/test_oracle_sampling.py).
- accept: closed form (sampler.py:451-452).
- speculative_verify (chain of k): pinned by exact enumeration of the
  losslessness invariant on tiny vocabularies and against the per-position
  restatement of the reference policy.
- apply_penalty: transformers' closed form; parity unpinned against SGLang's
  penalizer (sglang is not installed; the reference's own LoopSpec path
  rejects repetition_penalty != 1, server/loopspec_scheduler.py:141-148).
- top_k cutoff: only the joint top-k/top-p rule of distributions.py:72-86 is
  the reference's own; the top-k-only path calls sgl_kernel.top_k_renorm_prob
  (absent) -- parity unpinned for that path.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .numerics import (
    F32, F64, FX_BITS, LOG2E, exp2q, exp2q_k, fx46, floor_u_times, mass_to_f32, tree_sum_f32,
)


# ---------------------------------------------------------------------------
# (a) logit processing
# ---------------------------------------------------------------------------

def inv_f32(x: float) -> np.float32:
    """Binary32 reciprocal RN(1 / RN32(x))."""
    return F32(F32(1.0) / F32(x))


def apply_penalty(x: np.ndarray, history, penalty: float) -> np.ndarray:
    """Repetition penalty over a token history (transformers closed form).

    For every distinct token id in `history`: x < 0 -> x * penalty, else
    x * RN(1/penalty) (a division by a scalar is a multiplication by its
    binary32 reciprocal on the GPU torch path). Applied before temperature.
    """
    if penalty == 1.0 or history is None or len(history) == 0:
        return x
    x = x.copy()
    ids = np.unique(np.asarray(history, dtype=np.int64))
    v = x[ids]
    x[ids] = np.where(v < 0, (v * F32(penalty)).astype(F32), (v * inv_f32(penalty)).astype(F32))
    return x


@dataclass
class Processed:
    """Processed logits of one row: x = penalised logits, c = the binary32
    scale RN(LOG2E * RN(1/T)) applied inside the exponential, epv = elements
    per 16-byte vector of the logits' storage type (4 for float32, 8 for
    bfloat16 / float16), which fixes the summation order of the chunk masses."""
    x: np.ndarray
    c: np.float32
    epv: int = 4


def scale_of(temperature: float) -> np.float32:
    """c = RN(LOG2E * RN(1/T)); T == 1 gives LOG2E."""
    return F32(LOG2E * inv_f32(temperature))


def process_logits(logits: np.ndarray, temperature: float = 1.0, penalty: float = 1.0, history=None,
                   epv: int = 4) -> Processed:
    """Penalised logits and the temperature scale (distributions.py:44-48).

    The reference divides float32 logits by the temperature and takes
    softmax; here the temperature enters as the scale c of the base-2
    exponent (2^(c x) = e^(x / T)), so T == 1 and T != 1 share one path.
    """
    x = np.asarray(logits, dtype=F32).copy()
    x = apply_penalty(x, history, penalty)
    return Processed(x, scale_of(temperature), epv)


CHUNK = 2048  # elements per softmax chunk (a constant of the declared arithmetic)
LANES = 64    # lanes per chunk in the mass summation order
SCALE_SLOTS = 128  # chunks per row at most; the normaliser sums this many slots


@dataclass
class RowSoftmax:
    x: np.ndarray      # penalised logits
    c: np.float32      # exponent scale
    m: np.float32      # row max of the scaled chunk maxima, max_j mc_j
    e: np.ndarray      # exp2q(fma(x, c, -mc_j)), chunk-relative
    m_chunks: np.ndarray   # per-chunk max of x
    mc_chunks: np.ndarray  # RN(m_j * c)
    f_chunks: np.ndarray   # exp2q(RN(mc_j - m))
    mass_chunks: np.ndarray  # chunk masses M_j (binary32, fixed summation order)
    s: np.float32      # normaliser S
    g_chunks: np.ndarray   # RN(f_j / S)
    p: np.ndarray      # probabilities RN(e_i * g_j)


def chunk_mass(e_chunk: np.ndarray, epv: int) -> np.float32:
    """M_j of one chunk of CHUNK e-values (zero padded past the vocabulary).

    Summation order: the chunk is read as 16-byte vectors of epv elements;
    lane t of LANES owns vectors u * LANES + t (u = 0, 1, ...); each lane sums
    its 32 elements pairwise in (u, element) order, then the lane sums are
    summed pairwise in lane order.
    """
    nvc = CHUNK // (LANES * epv)
    lanes = np.asarray(e_chunk, dtype=F32).reshape(nvc, LANES, epv).transpose(1, 0, 2).reshape(LANES, nvc * epv)
    return F32(tree_sum_f32(tree_sum_f32(lanes)))


def softmax_row(x, c=None, epv: int = 4) -> RowSoftmax:
    """softmax(x / T) in the declared chunked arithmetic (distributions.py:44-48).

    x is a Processed row (or raw logits with T = 1). The row is cut into chunks
    of CHUNK elements. Chunk j: m_j = max x, mc_j = RN(m_j c),
    e_i = exp2q(fma(x_i, c, -mc_j)), M_j = chunk_mass(e). Row: m = max mc_j,
    f_j = exp2q(RN(mc_j - m)), S = pairwise sum over SCALE_SLOTS slots of
    RN(f_j M_j) (zero past the last chunk), g_j = RN(f_j / S),
    p_i = RN(e_i g_j). Every chunk can be processed on its own before the
    row-wide values are known, which is what lets the kernels read the logits
    once with many workgroups per row.
    """
    if isinstance(x, Processed):
        x, c, epv = x.x, x.c, x.epv
    c = LOG2E if c is None else F32(c)
    x = np.asarray(x, dtype=F32)
    v = len(x)
    nch = -(-v // CHUNK)
    if nch > SCALE_SLOTS:
        raise ValueError("vocabulary larger than SCALE_SLOTS chunks")
    xp = np.full(nch * CHUNK, -np.inf, dtype=F32)
    xp[:v] = x
    xc = xp.reshape(nch, CHUNK)
    with np.errstate(invalid="ignore", over="ignore"):
        m_chunks = np.max(xc, axis=1).astype(F32)
        mc = (m_chunks * c).astype(F32)
        t = _fma_rows(xc, c, (-mc).astype(F32))
        e = exp2q(t)
        mass = np.array([chunk_mass(e[j], epv) for j in range(nch)], dtype=F32)
        m = F32(np.max(mc))
        f = exp2q((mc - m).astype(F32))
        fm = np.zeros(SCALE_SLOTS, dtype=F32)
        fm[:nch] = (f * mass).astype(F32)
        s = F32(tree_sum_f32(fm))
        g = (f / s).astype(F32)
        p = (e * g[:, None]).astype(F32).reshape(-1)[:v]
    return RowSoftmax(x, c, m, e.reshape(-1)[:v], m_chunks, mc, f, mass, s, g, p)


def _fma_rows(xc: np.ndarray, c: np.float32, nmc: np.ndarray) -> np.ndarray:
    from .numerics import fma32
    return fma32(xc, np.full_like(xc, c), np.broadcast_to(nmc[:, None], xc.shape))


def p_at(soft: RowSoftmax, idx: int) -> np.float32:
    """p of one element recomputed from its logit (what the kernels do for a
    single token): RN(exp2q(fma(x, c, -mc_j)) * g_j)."""
    from .numerics import fma32
    j = idx // CHUNK
    t = fma32(soft.x[idx], soft.c, -soft.mc_chunks[j])
    return F32(exp2q(t) * soft.g_chunks[j])


def threshold_fx(top_p: float) -> int:
    return int(fx46(F32(top_p)))


def top_p_cutoff(p: np.ndarray, top_p: float) -> tuple[np.float32, int]:
    """Cutoff value and retained mass of the top-p rule (distributions.py:59-70).

    The reference sorts descending, takes the first sorted index whose
    cumulative mass reaches top_p (searchsorted, right=False, clamped to V-1)
    and keeps every probability >= the value found there (ties kept). With
    exact masses that is: c = max{v in p : sum_{p_i >= v} fx46(p_i) >= thr};
    if no v qualifies (rounding left total < thr), c = min(p).
    Returns (c, retained mass = sum_{p_i >= c} fx46(p_i)).
    """
    p = np.asarray(p, dtype=F32)
    w = fx46(p)
    thr = threshold_fx(top_p)
    vals, inv = np.unique(p, return_inverse=True)  # ascending unique values
    mass = np.zeros(len(vals), dtype=object)
    np.add.at(mass, inv, w.astype(object))
    cum = 0
    for j in range(len(vals) - 1, -1, -1):
        cum += int(mass[j])
        if cum >= thr:
            return F32(vals[j]), cum
    return F32(vals[0]), cum


def top_k_value(p: np.ndarray, top_k: int) -> np.float32:
    """k-th largest probability (distributions.py:81), counting duplicates."""
    return F32(np.sort(np.asarray(p, dtype=F32))[::-1][top_k - 1])


def retained_mass(p: np.ndarray, c: np.float32) -> int:
    p = np.asarray(p, dtype=F32)
    return int(fx46(np.where(p >= c, p, F32(0))).sum(dtype=np.uint64))


def normalize_retained(p: np.ndarray, c: np.float32, mass_fx: int) -> np.ndarray:
    """values >= c divided by the retained mass, else 0 (sampler.py:424)."""
    p = np.asarray(p, dtype=F32)
    mass = mass_to_f32(mass_fx)
    return np.where(p >= c, (p / mass).astype(F32), F32(0)).astype(F32)


@dataclass
class FilteredRow:
    soft: RowSoftmax
    cutoff: np.float32     # min(p) when unfiltered
    mass_fx: int
    P: np.ndarray          # filtered, renormalised (== p when unfiltered)
    filtered: bool


def filter_row(x, top_p: float, top_k: int = 0) -> FilteredRow:
    """filtered_probabilities for one processed-logit row (distributions.py:14-86).

    top_k == 0 (or >= V) and top_p == 1: the unfiltered softmax, returned as is.
    top-p only: cutoff from top_p_cutoff. Both: cutoff = max(k-th value, top-p
    cutoff), renormalised once. top-k only: p >= k-th value (parity unpinned).
    x is a Processed row or raw logits (T = 1).
    """
    soft = softmax_row(x)
    v = len(soft.p)
    eff_k = 0 if top_k >= v else top_k
    if eff_k == 0 and top_p >= 1.0:
        return FilteredRow(soft, F32(np.min(soft.p)), int(fx46(soft.p).sum(dtype=np.uint64)), soft.p, False)
    if eff_k == 0:
        c, mass = top_p_cutoff(soft.p, top_p)
    elif top_p >= 1.0:
        c = top_k_value(soft.p, eff_k)
        mass = retained_mass(soft.p, c)
    else:
        cp, _ = top_p_cutoff(soft.p, top_p)
        c = max(F32(top_k_value(soft.p, eff_k)), cp)
        mass = retained_mass(soft.p, c)
    return FilteredRow(soft, F32(c), mass, normalize_retained(soft.p, c, mass), True)


# ---------------------------------------------------------------------------
# (c) categorical sampling and acceptance
# ---------------------------------------------------------------------------

def categorical_pick(w: np.ndarray, u: float) -> int:
    """Inverse-CDF draw over weights in [0, 1] (sampler.py:22-102).

    The reference picks the first 2048-chunk whose cumulative mass exceeds
    u * total and then the first token in it whose cumulative mass exceeds the
    remaining target; with exact masses that is the first index j with
    sum_{i <= j} fx46(w_i) > floor(u * total). Zero total mass selects index 0,
    as the reference's all-false argmax does.
    """
    W = fx46(np.asarray(w, dtype=F32))
    total = int(W.sum(dtype=np.uint64))
    if total == 0:
        return 0
    target = floor_u_times(F32(u), total)
    cum = np.cumsum(W, dtype=np.uint64)
    return int(np.argmax(cum > np.uint64(target)))


def accept(u: float, p_x: float, q_x: float) -> bool:
    """u < min(1, p/q) in binary32 (sampler.py:451-452); a NaN ratio rejects."""
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = F32(F32(p_x) / F32(q_x))
    if np.isnan(ratio):
        return False
    return bool(F32(u) < min(F32(1.0), ratio))


def residual(P: np.ndarray, Q: np.ndarray) -> tuple[np.ndarray, bool]:
    """normalize(max(P - Q, 0)), falling back to normalize(P) at zero mass.

    Follows sglang_recurrent/loopspec/sampling/rejection.py:60-69.
    Returns (distribution, used_fallback).
    """
    P = np.asarray(P, dtype=F32)
    Q = np.asarray(Q, dtype=F32)
    d = np.maximum((P - Q).astype(F32), F32(0)).astype(F32)
    d_fx = int(fx46(d).sum(dtype=np.uint64))
    if d_fx > 0:
        return (d / mass_to_f32(d_fx)).astype(F32), False
    p_fx = int(fx46(P).sum(dtype=np.uint64))
    pm = mass_to_f32(p_fx) if p_fx > 0 else F32(1.0)
    return (P / pm).astype(F32), True


@dataclass
class SpecResult:
    accept_len: np.ndarray   # int32 [B]
    tokens: np.ndarray       # int64 [B, k+1], -1 padded
    cutoffs: np.ndarray      # float32 [B, 2k+1] per-row cutoff (target rows then draft rows)
    masses: np.ndarray       # uint64 [B, 2k+1] retained masses
    maxes: np.ndarray        # float32 [B, 2k+1] row max of the scaled chunk maxima
    norms: np.ndarray        # float32 [B, 2k+1] normalisers S


def speculative_verify(target_logits, draft_logits, draft_tokens, uniforms, temperature=1.0,
                       top_p=1.0, penalty=1.0, histories=None, top_k=0, epv=4) -> SpecResult:
    """Lossless speculative verification over a chain of k draft positions.

    Per position i the reference's q1 rule (sampler.py:428-460): accept the
    draft token x_i iff u[b,i] < min(1, P_i[x_i] / Q_i[x_i]); on the first
    rejection emit a sample of normalize(max(P_i - Q_i, 0)) (fallback
    normalize(P_i), rejection.py:60-69) drawn with u[b, k+i]; if all k accept,
    emit a bonus sample of P_k drawn with u[b, 2k] (the direct final sample of
    policy.py:156-165). P and Q are the filtered distributions of the target
    and draft rows after penalty / temperature / top-p (distributions.py:89-149).
    Positions after a rejection are discarded (pipeline.py:379-412).

    target_logits [B, k+1, V], draft_logits [B, k, V] (any float dtype, taken
    as binary32), draft_tokens int64 [B, k], uniforms float32 [B, 2k+1];
    epv = 4 for float32 logits, 8 for bfloat16 / float16 (see Processed).
    """
    t = np.asarray(target_logits, dtype=F32)
    d = np.asarray(draft_logits, dtype=F32)
    xs = np.asarray(draft_tokens, dtype=np.int64)
    u = np.asarray(uniforms, dtype=F32)
    b_n, kp1, _ = t.shape
    k = kp1 - 1
    acc = np.zeros(b_n, dtype=np.int32)
    tok = np.full((b_n, kp1), -1, dtype=np.int64)
    cut = np.zeros((b_n, 2 * k + 1), dtype=F32)
    mas = np.zeros((b_n, 2 * k + 1), dtype=np.uint64)
    mx = np.zeros((b_n, 2 * k + 1), dtype=F32)
    nrm = np.zeros((b_n, 2 * k + 1), dtype=F32)
    for b in range(b_n):
        hist = None if histories is None else histories[b]
        rows_t = [filter_row(process_logits(t[b, i], temperature, penalty, hist, epv), top_p, top_k)
                  for i in range(kp1)]
        rows_d = [filter_row(process_logits(d[b, i], temperature, penalty, hist, epv), top_p, top_k)
                  for i in range(k)]
        for j, r in enumerate(rows_t + rows_d):
            cut[b, j], mas[b, j], mx[b, j], nrm[b, j] = r.cutoff, r.mass_fx, r.soft.m, r.soft.s
        a = 0
        while a < k:
            x = int(xs[b, a])
            if not accept(u[b, a], rows_t[a].P[x], rows_d[a].P[x]):
                break
            tok[b, a] = x
            a += 1
        if a < k:
            dist, _ = residual(rows_t[a].P, rows_d[a].P)
            tok[b, a] = categorical_pick(dist, u[b, k + a])
        else:
            tok[b, a] = categorical_pick(rows_t[k].P, u[b, 2 * k])
        acc[b] = a
    return SpecResult(acc, tok, cut, mas, mx, nrm)


# ---------------------------------------------------------------------------
# Drop-in level restatements (dense rows), used by the sampler API tests.
# ---------------------------------------------------------------------------

def filtered_probabilities(logits: np.ndarray, temperature: float, top_k: int, top_p, top_p_thresholds=None,
                           epv: int = 4):
    """distributions.py:14-86 over [B, V]; per-row thresholds optional."""
    logits = np.asarray(logits, dtype=F32)
    out = np.zeros_like(logits)
    for b in range(logits.shape[0]):
        tp = float(top_p_thresholds[b]) if top_p_thresholds is not None and top_p < 1 else top_p
        out[b] = filter_row(process_logits(logits[b], temperature, epv=epv), tp, top_k).P
    return out


def sample_rows(probs: np.ndarray, uniforms: np.ndarray) -> np.ndarray:
    """CategoricalSampler.sample with supplied uniforms (sampler.py:508-588)."""
    return np.array([categorical_pick(probs[b], uniforms[b]) for b in range(probs.shape[0])], dtype=np.int64)


def sample_top_p_rows(probs, cutoffs, uniforms, sample_rows_idx=None) -> np.ndarray:
    """sample_top_p: draw from unnormalised retained weights p >= cutoff (sampler.py:105-175)."""
    probs = np.asarray(probs, dtype=F32)
    rows = range(probs.shape[0]) if sample_rows_idx is None else [int(r) for r in sample_rows_idx]
    out = []
    for s, r in enumerate(rows):
        w = np.where(probs[r] >= F32(cutoffs[r]), probs[r], F32(0))
        out.append(categorical_pick(w, uniforms[s]))
    return np.array(out, dtype=np.int64)


def conditional_residual(first, second, selected, uniforms):
    """sample_conditional_residual (sampler.py:178-344, 629-703).

    r = max(q2 - q1, 0) with r[x1] = 0; candidate y drawn from unnormalised r
    with u; R = r / mass (zero row at zero mass); action = (mass > 0) and
    q2[x1] < q1[x1]. Returns (R, actions, ids).
    """
    first = np.asarray(first, dtype=F32)
    second = np.asarray(second, dtype=F32)
    b_n, _ = first.shape
    R = np.zeros_like(first)
    act = np.zeros(b_n, dtype=np.int64)
    ids = np.zeros(b_n, dtype=np.int64)
    for b in range(b_n):
        x1 = int(selected[b])
        r = np.maximum((second[b] - first[b]).astype(F32), F32(0)).astype(F32)
        r[x1] = 0
        ids[b] = categorical_pick(r, uniforms[b])
        m_fx = int(fx46(r).sum(dtype=np.uint64))
        if m_fx > 0:
            R[b] = (r / mass_to_f32(m_fx)).astype(F32)
        act[b] = int(m_fx > 0 and second[b, x1] < first[b, x1])
    return R, act, ids


def verify_decisions(target_masses, proposal_masses, tokens, uniforms) -> np.ndarray:
    """CategoricalSampler.verify 5-tuples (sampler.py:428-460, 705-735)."""
    n = len(tokens)
    out = np.zeros((n, 5), dtype=np.int64)
    for i in range(n):
        a = accept(uniforms[i], target_masses[i], proposal_masses[i])
        out[i] = (int(tokens[i]) if a else -1, 0, int(a), int(not a), 0)
    return out


def rejection_run(first, target, second, token: int, has_second: bool, u0: float, u1: float):
    """RejectionSampler._run for one rejected q1 (rejection.py:42-97).

    F = normalize(max(P - Q1, 0)) (fallback normalize(P)); with q2 accept y iff
    u0 < min(1, F[y] / R[y]); the fallback sample always consumes u1 from
    normalize(max(F - R, 0)) (or F without q2 / at zero mass).
    Returns (token, second_accepted, second_rejected).
    """
    F, _ = residual(target, first)
    if has_second:
        a = accept(u0, F[token], np.asarray(second, dtype=F32)[token])
    else:
        a = False
    if has_second:
        d = np.maximum((F - np.asarray(second, dtype=F32)).astype(F32), F32(0)).astype(F32)
        d_fx = int(fx46(d).sum(dtype=np.uint64))
        fallback = (d / mass_to_f32(d_fx)).astype(F32) if d_fx > 0 else F
    else:
        fallback = F
    sampled = categorical_pick(fallback, u1)
    return (int(token) if a else sampled, int(a), int(has_second and not a))


__all__ = [n for n in dir() if not n.startswith("_")] + ["FX_BITS", "F64", "exp2q", "CHUNK"]
