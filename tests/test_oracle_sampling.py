"""Pin the sampling oracle: torch-CPU restatements, brute force, closed forms, losslessness."""

import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sampling as os_
from oracle import torch_ref


def test_softmax_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 49152, generator=g) * 3
    for r in range(8):
        soft = os_.softmax_row(x[r].numpy())
        ref64 = torch.softmax(x[r].double(), -1).numpy()
        ref32 = torch.softmax(x[r], -1).numpy()
        big = ref64 > 1e-30
        # x - max is rounded to binary32 first (as torch's fp32 softmax does): for
        # |x - max| ~ 24 that alone is ~1e-6 relative in exp(.)
        assert np.max(np.abs(soft.p[big] - ref64[big]) / ref64[big]) < 3e-6
        assert np.max(np.abs(soft.p[big] - ref32[big]) / ref32[big]) < 1e-5  # the contract tolerance


def test_chunk_mass_order():
    # M_j sums each lane's 32 elements pairwise, lane t owning 16-byte vectors
    # u * 64 + t; placing two 2^-24 next to a 1 in one pairwise group loses
    # them (ties to even), placing them in a group of their own keeps 2^-23.
    tiny = np.float32(2.0 ** -24)
    for epv in (4, 8):
        e = np.zeros(os_.CHUNK, np.float32)
        e[0], e[1], e[2] = 1, tiny, tiny          # lane 0: (1 + t) + (t + 0) -> 1
        assert os_.chunk_mass(e, epv) == np.float32(1)
        e = np.zeros(os_.CHUNK, np.float32)
        e[0], e[epv], e[epv + 1] = 1, tiny, tiny  # the tiny pair is lane 1's first vector
        assert os_.chunk_mass(e, epv) == np.float32(1 + 2.0 ** -23)
    # Elements 1024 and 1028: with epv = 4 they open lane 0's and lane 1's
    # fifth vectors (each tiny meets the 1 on its own and is lost); with epv = 8
    # both sit in lane 0's third vector and add up first.
    e = np.zeros(os_.CHUNK, np.float32)
    e[0], e[1024], e[1028] = 1, tiny, tiny
    assert os_.chunk_mass(e, 4) == np.float32(1)
    assert os_.chunk_mass(e, 8) == np.float32(1 + 2.0 ** -23)


def test_chunked_softmax_closed_forms():
    c = os_.CHUNK
    # A zero row of 3 chunks + 5: every e = 1, M = (2048, 2048, 2048, 5),
    # S = V exactly, p = RN(1 / V).
    v = 3 * c + 5
    soft = os_.softmax_row(np.zeros(v, np.float32))
    assert np.array_equal(soft.mass_chunks, np.float32([c, c, c, 5])) and soft.s == np.float32(v)
    assert np.all(soft.p == np.float32(1) / np.float32(v))
    # Zeros next to a maximum whose scaled value rounds to 1: t = -1 exactly,
    # so their e is exactly 1/2.
    x = np.zeros(c, np.float32)
    x[0] = np.float32(1.0) / nm.LOG2E
    soft = os_.softmax_row(x)
    assert soft.mc_chunks[0] == 1 and soft.e[0] == 1 and np.all(soft.e[1:] == np.float32(0.5))
    # A chunk of -inf contributes nothing and the others are unaffected; the
    # maximum may sit in any chunk.
    x = (np.random.default_rng(2).standard_normal(3 * c) * 2).astype(np.float32)
    x[c:2 * c] = -np.inf
    x[2 * c + 7] = 30.0
    soft = os_.softmax_row(x)
    assert soft.f_chunks[1] == 0 and soft.mass_chunks[1] == 0 and not soft.p[c:2 * c].any()
    assert soft.f_chunks[2] == 1 and soft.p.argmax() == 2 * c + 7
    ref = torch.softmax(torch.from_numpy(x).double(), -1).numpy()
    big = ref > 1e-30
    assert np.max(np.abs(soft.p[big] - ref[big]) / ref[big]) < 3e-6
    # The normaliser is sum_j f_j M_j to binary32 accuracy, and p sums to 1.
    s64 = sum(float(soft.f_chunks[j]) * float(soft.mass_chunks[j]) for j in range(3))
    assert abs(float(soft.s) / s64 - 1) < 1e-6
    assert abs(float(soft.p.astype(np.float64).sum()) - 1.0) < 1e-5
    # p of a single element recomputed from its logit is the row's value.
    for i in (0, 5, c + 3, 2 * c + 7, 3 * c - 1):
        assert os_.p_at(soft, i) == soft.p[i]


def test_softmax_layouts_and_temperature_agree_with_torch():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 128256, generator=g) * 4
    for r in range(2):
        for epv, temp in ((4, 1.0), (8, 0.7)):
            soft = os_.softmax_row(os_.process_logits(x[r].numpy(), temp, epv=epv))
            ref = torch.softmax(x[r].double() / temp, -1).numpy()
            big = ref > 1e-30
            assert np.max(np.abs(soft.p[big] - ref[big]) / ref[big]) < 1e-5


def test_temperature_and_penalty_closed_form():
    x = np.float32([-2.0, -0.5, 0.0, 0.5, 3.0])
    y = os_.process_logits(x, temperature=0.7, penalty=1.1, history=[0, 3, 3, 4])
    inv_r = np.float32(1) / np.float32(1.1)
    want = np.float32([np.float32(-2.0 * np.float32(1.1)), -0.5, 0.0, np.float32(0.5 * inv_r), np.float32(3.0 * inv_r)])
    assert np.array_equal(y.x, want)
    assert y.c == np.float32(nm.LOG2E * (np.float32(1) / np.float32(0.7)))
    assert np.array_equal(os_.process_logits(x, 1.0).x, x) and os_.process_logits(x, 1.0).c == nm.LOG2E


def brute_cutoff(p, top_p):
    """sort -> exact cumsum -> first index reaching thr (clamped) -> keep p >= value."""
    w = [int(v) for v in nm.fx46(p)]
    order = sorted(range(len(p)), key=lambda i: -float(p[i]))
    thr = os_.threshold_fx(top_p)
    cum = 0
    idx = len(p) - 1
    for j, i in enumerate(order):
        cum += w[i]
        if cum >= thr:
            idx = j
            break
    c = p[order[idx]]
    return c, sum(w[i] for i in range(len(p)) if p[i] >= c)


@pytest.mark.parametrize("seed", range(40))
def test_top_p_cutoff_bruteforce_tiny(seed):
    rng = np.random.default_rng(seed)
    v = int(rng.integers(1, 13))
    logits = rng.integers(-3, 4, size=v).astype(np.float32)  # many equal values
    p = os_.softmax_row(logits).p
    for top_p in [0.05, 0.3, 0.5, 0.7, 0.9, 0.999, 1.0]:
        assert os_.top_p_cutoff(p, top_p) == brute_cutoff(p, top_p)


def test_top_p_special_cases():
    p = os_.softmax_row(np.float32([1, 2, 3, 3, 0])).p
    # top_p -> 0+: the max and its ties
    c, _ = os_.top_p_cutoff(p, 1e-9)
    assert c == p.max() and (p >= c).sum() == 2
    # all-equal row keeps everything
    q = os_.softmax_row(np.zeros(7, np.float32)).p
    c, m = os_.top_p_cutoff(q, 0.5)
    assert (q >= c).all() and m == int(nm.fx46(q).sum())
    # threshold above the representable total: clamp to the last sorted value (the minimum)
    c, _ = os_.top_p_cutoff(p, 1.0)
    assert c == p.min() or int(nm.fx46(p).sum()) >= os_.threshold_fx(1.0)
    # a run of equal values straddling the threshold is kept whole
    r = np.float32([0.4, 0.2, 0.2, 0.2])
    c, m = os_.top_p_cutoff(r, 0.5)
    assert c == np.float32(0.2) and m == int(nm.fx46(r).sum())


@pytest.mark.parametrize("temperature,top_p", [(1.0, 0.7), (0.7, 0.9), (1.3, 0.5)])
def test_filter_matches_torch_reference(temperature, top_p):
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(6, 49152, generator=g) * 3
    ref = torch_ref.filtered_probabilities(logits, temperature, 1 << 30, top_p).numpy()
    got = os_.filtered_probabilities(logits.numpy(), temperature, 1 << 30, top_p)
    assert np.array_equal(ref > 0, got > 0)  # identical retained sets
    nz = ref > 0
    assert np.max(np.abs(got[nz] - ref[nz]) / ref[nz]) < 2e-6


def test_joint_top_k_top_p_matches_torch_reference():
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(4, 4096, generator=g) * 2
    for top_k in [1, 5, 50, 4000]:
        ref = torch_ref.filtered_probabilities(logits, 1.0, top_k, 0.8).numpy()
        got = os_.filtered_probabilities(logits.numpy(), 1.0, top_k, 0.8)
        assert np.array_equal(ref > 0, got > 0), top_k
        nz = ref > 0
        assert np.max(np.abs(got[nz] - ref[nz]) / ref[nz]) < 2e-6


def test_categorical_pick_matches_torch_reference():
    g = torch.Generator().manual_seed(5)
    probs = torch.softmax(torch.randn(64, 5000, generator=g) * 2, -1)
    u = torch.rand(64, generator=g)
    ref = torch_ref.categorical_pick(probs, u).numpy()
    got = os_.sample_rows(probs.numpy(), u.numpy())
    assert np.array_equal(ref, got)


def test_categorical_pick_closed_forms():
    w = np.zeros(5000, np.float32)
    w[2047], w[2048] = 0.5, 0.5
    assert os_.categorical_pick(w, 0.0) == 2047  # u = 0: first positive-mass token
    assert os_.categorical_pick(w, 0.4999999) == 2047
    assert os_.categorical_pick(w, 0.5) == 2048  # chunk boundary, strict '>'
    one = np.zeros(10, np.float32)
    one[7] = 1.0
    assert all(os_.categorical_pick(one, u) == 7 for u in [0.0, 0.3, 0.9999999])
    assert os_.categorical_pick(np.zeros(10, np.float32), 0.5) == 0  # zero mass -> index 0
    w = np.float32([0.25, 0, 0, 0.75])  # zero-mass middle
    assert os_.categorical_pick(w, 0.2) == 0 and os_.categorical_pick(w, 0.25) == 3


def test_categorical_pick_frequencies_chi_square():
    from scipy.stats import chisquare

    rng = np.random.default_rng(6)
    p = os_.softmax_row(rng.standard_normal(20).astype(np.float32)).p
    from loopspec_amd import philox

    u = philox.uniforms((200000,), seed=11)
    counts = np.bincount([os_.categorical_pick(p, x) for x in u[:40000]], minlength=20)
    pe = p.astype(np.float64)
    assert chisquare(counts, pe / pe.sum() * counts.sum()).pvalue > 1e-4


def test_verify_rule_closed_form():
    assert os_.accept(0.5, 0.3, 0.5)          # 0.5 < 0.6
    assert not os_.accept(0.6, 0.3, 0.5)      # strict '<'
    assert os_.accept(0.99999994, 0.9, 0.1)   # ratio > 1 -> min(1, .) = 1
    assert not os_.accept(0.0, 0.0, 0.0)      # NaN ratio rejects
    dec = os_.verify_decisions([0.3, 0.3], [0.5, 0.5], [7, 9], np.float32([0.5, 0.6]))
    assert dec.tolist() == [[7, 0, 1, 0, 0], [-1, 0, 0, 1, 0]]
    ref = torch_ref.verify(torch.tensor([0.3, 0.3]), torch.tensor([0.5, 0.5]), torch.tensor([7, 9]),
                           torch.tensor([0.5, 0.6]))
    assert ref.tolist() == dec.tolist()


def exact_emitted_distribution(P, Q):
    """Exact marginal of the emitted token for one position of speculative sampling."""
    v = len(P)
    out = [Fraction(0)] * v
    d = [max(P[i] - Q[i], Fraction(0)) for i in range(v)]
    dm = sum(d)
    res = [x / dm for x in d] if dm > 0 else [x / sum(P) for x in P]
    for x in range(v):
        if Q[x] == 0:
            continue
        a = min(Fraction(1), P[x] / Q[x])
        out[x] += Q[x] * a
        for y in range(v):
            out[y] += Q[x] * (1 - a) * res[y]
    return out


@pytest.mark.parametrize("seed", range(10))
def test_losslessness_exact_enumeration(seed):
    """The accept/residual rule emits exactly P for any draft distribution Q."""
    rng = np.random.default_rng(seed)
    v = int(rng.integers(2, 7))
    pw = [Fraction(int(x)) for x in rng.integers(0, 5, v)]
    qw = [Fraction(int(x)) for x in rng.integers(0, 5, v)]
    if sum(pw) == 0:
        pw[0] = Fraction(1)
    if sum(qw) == 0:
        qw[-1] = Fraction(1)
    P = [x / sum(pw) for x in pw]
    Q = [x / sum(qw) for x in qw]
    assert exact_emitted_distribution(P, Q) == P


def test_speculative_verify_statistically_lossless():
    """Declared-arithmetic chain verify: emitted first token ~ P_0 (chi-square)."""
    from scipy.stats import chisquare
    from loopspec_amd import philox

    rng = np.random.default_rng(7)
    v = 12
    tl = (rng.standard_normal((1, 2, v)) * 1.5).astype(np.float32)
    dl = (tl[:, :1] + rng.standard_normal((1, 1, v))).astype(np.float32)
    P0 = os_.filter_row(tl[0, 0], 1.0).P
    Q0 = os_.filter_row(dl[0, 0], 1.0).P
    n = 6000
    uq = philox.uniforms((n,), seed=21)
    uv = philox.uniforms((n, 3), seed=22)
    counts = np.zeros(v)
    for i in range(n):
        x = os_.categorical_pick(Q0, uq[i])
        res = os_.speculative_verify(tl, dl, np.array([[x]]), uv[i:i + 1])
        counts[res.tokens[0, 0]] += 1
    pe = P0.astype(np.float64)
    assert chisquare(counts, pe / pe.sum() * counts.sum()).pvalue > 1e-4


@pytest.mark.parametrize("temperature,top_p", [(1.0, 0.7), (0.8, 0.95)])
def test_speculative_verify_matches_torch_reference(temperature, top_p):
    from loopspec_amd import philox

    g = torch.Generator().manual_seed(8)
    b, k, v = 6, 2, 8192
    target = torch.randn(b, k + 1, v, generator=g) * 3
    draft = target[:, :k] + torch.randn(b, k, v, generator=g)
    q = torch_ref.filtered_probabilities(draft.reshape(b * k, v), temperature, 1 << 30, top_p)
    du = torch.from_numpy(philox.uniforms((b * k,), seed=3))
    drafts = torch_ref.categorical_pick(q, du).reshape(b, k)
    u = torch.from_numpy(philox.uniforms((b, 2 * k + 1), seed=4))
    a_ref, t_ref = torch_ref.speculative_verify(target, draft, drafts, u, temperature, top_p)
    res = os_.speculative_verify(target.numpy(), draft.numpy(), drafts.numpy(), u.numpy(), temperature, top_p)
    assert np.array_equal(res.accept_len, a_ref.numpy())
    assert np.array_equal(res.tokens, t_ref.numpy())


def test_rejection_run_matches_torch_reference():
    g = torch.Generator().manual_seed(9)
    v = 3000
    for case in range(6):
        P = torch.softmax(torch.randn(v, generator=g) * 2, -1)
        Q1 = torch.softmax(torch.randn(v, generator=g) * 2, -1)
        R = torch.softmax(torch.randn(v, generator=g) * 2, -1)
        y = int(torch.randint(0, v, (1,), generator=g))
        u0, u1 = float(torch.rand(1, generator=g)), float(torch.rand(1, generator=g))
        has = case % 2 == 0
        want = torch_ref.rejection_run(Q1, P, R, y, has, u0, u1)
        got = os_.rejection_run(Q1.numpy(), P.numpy(), R.numpy(), y, has, np.float32(u0), np.float32(u1))
        assert got == want


def test_conditional_residual_matches_triton_restatement():
    g = torch.Generator().manual_seed(10)
    b, v = 5, 4000
    q1 = torch.softmax(torch.randn(b, v, generator=g), -1)
    q2 = torch.softmax(torch.randn(b, v, generator=g), -1)
    x1 = torch.randint(0, v, (b,), generator=g)
    q2[0] = q1[0]  # zero residual row -> action 0, zero distribution
    u = torch.rand(b, generator=g)
    R, act, ids = os_.conditional_residual(q1.numpy(), q2.numpy(), x1.numpy(), u.numpy())
    r = (q2 - q1).clamp_min(0)
    r[torch.arange(b), x1] = 0
    mass = r.sum(-1)
    want_R = torch.where(mass[:, None] > 0, r / mass[:, None], torch.zeros_like(r))
    want_act = ((mass > 0) & (q2[torch.arange(b), x1] < q1[torch.arange(b), x1])).long()
    assert np.array_equal(act, want_act.numpy())
    assert np.allclose(R, want_R.numpy(), rtol=2e-6, atol=1e-12)
    assert np.array_equal(ids[1:], torch_ref.categorical_pick(r[1:], u[1:]).numpy())
    assert act[0] == 0 and (R[0] == 0).all()


def test_penalised_speculative_verify_matches_torch_reference():
    """The repetition penalty in both restatements (x * RN(1/r) vs x / r differ
    by at most an ulp) leaves accept lengths and tokens equal on seeded rows."""
    from loopspec_amd import philox

    g = torch.Generator().manual_seed(9)
    b, k, v = 4, 3, 8192
    target = torch.randn(b, k + 1, v, generator=g) * 4
    draft = target[:, :k] + torch.randn(b, k, v, generator=g)
    hists = [torch.randint(0, v, (int(n),), generator=g) for n in (50, 400, 1, 2000)]
    x = torch.randn(3, v, generator=g) * 4
    pt = torch_ref.apply_penalty(x, hists[1], 1.1)
    po = np.stack([os_.apply_penalty(x[r].numpy(), hists[1].numpy(), 1.1) for r in range(3)])
    assert np.allclose(pt.numpy(), po, rtol=2e-7, atol=0)
    drafts = torch.zeros(b, k, dtype=torch.int64)
    du = torch.from_numpy(philox.uniforms((b, k), seed=5))
    for i in range(b):
        q = torch_ref.filtered_probabilities(torch_ref.apply_penalty(draft[i], hists[i], 1.1), 0.7, 1 << 30, 0.9)
        drafts[i] = torch_ref.categorical_pick(q, du[i])
    u = torch.from_numpy(philox.uniforms((b, 2 * k + 1), seed=6))
    a_ref, t_ref = torch_ref.speculative_verify(target, draft, drafts, u, 0.7, 0.9, 1.1, hists)
    res = os_.speculative_verify(target.numpy(), draft.numpy(), drafts.numpy(), u.numpy(), 0.7, 0.9, 1.1,
                                 [h.numpy() for h in hists])
    assert np.array_equal(res.accept_len, a_ref.numpy())
    assert np.array_equal(res.tokens, t_ref.numpy())
