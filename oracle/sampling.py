"""Sampling-path oracle on the declared arithmetic (numpy + C core; test infrastructure).

Every function restates one reference function; the docstring cites it. Rows
are processed independently. "p" is a softmax probability, "P" a filtered and
renormalised probability; masses are exact 2^-46 fixed-point integers (see
oracle.numerics). The softmax itself (chunk masses, row normaliser, p of each
logit) is computed by the C core oracle/native/ls_oracle.c. Parity status per
function:

- softmax_row, top_p_cutoff, filter_row, categorical_pick: pinned against
  torch-CPU restatements (oracle.torch_ref) on seeded inputs at the full
  BASELINE shapes, against the exact softmax in binary64, brute force on tiny
  vocabularies, tie/monotonicity invariants and closed-form special cases
  (tests/test_oracle_sampling.py).
- accept: closed form (sampler.py:451-452).
- speculative_verify (chain of k): pinned by exact enumeration of the
  losslessness invariant on tiny vocabularies and against the per-position
  restatement of the reference policy (oracle.torch_ref.speculative_verify)
  at the full C3/C4 shapes.
- apply_penalty: transformers' closed form x < 0 ? x * r : x / r, bit-equal
  to oracle.torch_ref.apply_penalty; parity unpinned against SGLang's
  penalizer (sglang is not installed; the reference's own LoopSpec path
  rejects repetition_penalty != 1, server/loopspec_scheduler.py:141-148).
- top_k cutoff: only the joint top-k/top-p rule of distributions.py:72-86 is
  the reference's own; the top-k-only path calls sgl_kernel.top_k_renorm_prob
  (absent). Its support is pinned to the k largest for distinct values and
  its weights to the renormalised p (tests/test_oracle_sampling.py); ties at
  the k-th value are kept by this build's convention, and parity with
  top_k_renorm_prob on ties stays unpinned.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import native
from .numerics import (
    F32, F64, FX_BITS, LOG2E, exp2m, exp2p, fx46, floor_u_times, mass_to_f32, scale_of, tree_sum_f32,
)


# ---------------------------------------------------------------------------
# (a) logit processing
# ---------------------------------------------------------------------------

def history_mask(history, vocab: int) -> np.ndarray:
    """Flags of the distinct in-vocabulary token ids of a history."""
    m = np.zeros(vocab, dtype=bool)
    if history is not None and len(history):
        ids = np.asarray(history, dtype=np.int64)
        ids = ids[(ids >= 0) & (ids < vocab)]
        m[ids] = True
    return m


def apply_penalty(x: np.ndarray, history, penalty: float) -> np.ndarray:
    """Repetition penalty over a token history (transformers' closed form,
    generation/logits_process.py:409-412): for every distinct token id of the
    history, x < 0 -> RN(x * r), else RN(x / r) with r the binary32 penalty.
    Applied before temperature."""
    x = np.asarray(x, dtype=F32)
    if penalty == 1.0 or history is None or len(history) == 0:
        return x.copy()
    return native.penalise(x, history_mask(history, len(x)), penalty)


@dataclass
class Processed:
    """Processed logits of one row: x = penalised logits, (cd, c) = the
    temperature scale (binary64, binary32), epv = elements per 16-byte
    vector of the logits' storage type (4 for float32, 8 for bfloat16 /
    float16), which fixes the summation order of the chunk masses, and pen =
    the flags of the penalised tokens (None without a penalty): they form a
    sub-chunk of their own in every chunk."""
    x: np.ndarray
    cd: float
    c: np.float32
    epv: int = 4
    pen: np.ndarray | None = None


def process_logits(logits: np.ndarray, temperature: float = 1.0, penalty: float = 1.0, history=None,
                   epv: int = 4) -> Processed:
    """Penalised logits and the temperature scale (distributions.py:44-48).

    The reference divides float32 logits by the temperature and takes
    softmax; here the temperature enters as the scale of the base-2 exponent
    (2^(cd x) = e^(x / T)), so T == 1 and T != 1 share one path.
    """
    x = np.asarray(logits, dtype=F32)
    cd, c = scale_of(temperature)
    if penalty != 1.0 and history is not None and len(history):
        pen = history_mask(history, len(x))
        return Processed(native.penalise(x, pen, penalty), cd, c, epv, pen)
    return Processed(x.copy(), cd, c, epv, None)


CHUNK = 2048  # elements per softmax chunk (a constant of the declared arithmetic)
LANES = 64    # lanes per chunk in the mass summation order
MAX_CHUNKS = 128  # chunks per row at most (vocabulary <= 262144)


@dataclass
class RowSoftmax:
    x: np.ndarray          # processed logits
    cd: float              # binary64 exponent scale
    c: np.float32          # binary32 exponent scale
    mcmax: np.float32      # row max of the scaled sub-chunk maxima
    s: np.float32          # normaliser S
    m_chunks: np.ndarray   # per-chunk max of the non-penalised x (m_j)
    mass_chunks: np.ndarray  # M_j
    pm_chunks: np.ndarray  # per-chunk max of the penalised x (pm_j)
    pmass_chunks: np.ndarray  # PM_j
    p: np.ndarray          # probabilities p(x_i)

    @property
    def mc_chunks(self) -> np.ndarray:
        return (self.m_chunks * self.c).astype(F32)

    @property
    def pmc_chunks(self) -> np.ndarray:
        return (self.pm_chunks * self.c).astype(F32)


def softmax_row(x, c=None, epv: int = 4) -> RowSoftmax:
    """softmax(x / T) in the declared arithmetic (distributions.py:44-48).

    x is a Processed row (or raw logits with T = 1). The row is cut into
    chunks of CHUNK elements; each chunk's non-penalised and penalised tokens
    give a (max, mass) pair each, relative to their own max, so every chunk
    can be reduced on its own before the row-wide values are known. The row
    normaliser S combines them, and every probability is then a function of
    its processed logit alone: p(x) = RN(exp2p(RN32(fma64(x, cd, -mcmax))) / S)
    (oracle/native/ls_oracle.c states the arithmetic in full).
    """
    if isinstance(x, Processed):
        pr = x
    else:
        cd, cf = scale_of(1.0) if c is None else (float(c), F32(c))
        pr = Processed(np.asarray(x, dtype=F32), cd, cf, epv, None)
    if -(-len(pr.x) // CHUNK) > MAX_CHUNKS:
        raise ValueError("vocabulary larger than MAX_CHUNKS chunks")
    p, mcmax, s, ch = native.row_softmax(pr.x, pr.cd, pr.epv, pr.pen)
    return RowSoftmax(pr.x, pr.cd, pr.c, mcmax, s, ch[:, 0].copy(), ch[:, 1].copy(), ch[:, 2].copy(),
                      ch[:, 3].copy(), p)


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


def p_of(soft: RowSoftmax, x) -> np.ndarray:
    """p of arbitrary processed logits under the row's constants."""
    return native.p_of(x, soft.cd, soft.mcmax, soft.s)


def p_at(soft: RowSoftmax, idx: int) -> np.float32:
    """p of one element recomputed from its logit (what the kernels do for a
    single token)."""
    return F32(p_of(soft, soft.x[idx : idx + 1])[0])


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
    order = np.argsort(-p, kind="stable")  # descending values
    cum = np.cumsum(w[order], dtype=np.uint64)  # exact: the total is below 2^47
    idx = int(np.searchsorted(cum, np.uint64(thr), side="left"))
    if idx >= len(p):
        return F32(p.min()), int(cum[-1])
    c = F32(p[order[idx]])
    return c, int(w[p >= c].sum(dtype=np.uint64))


def top_k_value(p: np.ndarray, top_k: int) -> np.float32:
    """k-th largest probability (distributions.py:81), counting duplicates."""
    return F32(np.sort(np.asarray(p, dtype=F32))[::-1][top_k - 1])


def retained_mass(p: np.ndarray, c: np.float32) -> int:
    p = np.asarray(p, dtype=F32)
    return int(fx46(np.where(p >= c, p, F32(0))).sum(dtype=np.uint64))


def normalize_retained(p: np.ndarray, c: np.float32, mass_fx: int) -> np.ndarray:
    """values >= c divided by the retained mass, else 0 (sampler.py:424); a
    row whose retained mass is 0 (no finite logit) filters to all zeros."""
    p = np.asarray(p, dtype=F32)
    if mass_fx == 0:
        return np.zeros_like(p)
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
            cut[b, j], mas[b, j], mx[b, j], nrm[b, j] = r.cutoff, r.mass_fx, r.soft.mcmax, r.soft.s
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


__all__ = [n for n in dir() if not n.startswith("_")] + ["FX_BITS", "F64", "exp2m", "exp2p", "CHUNK"]
