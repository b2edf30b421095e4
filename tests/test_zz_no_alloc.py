"""ls_spec_verify_noalloc (static scratch, allocates nothing) against ls_spec_verify.

Both entry points are called through the C-ABI on the same inputs and must give
identical accepted lengths and tokens. The no-allocation calls run twice in a
row, the second on a smaller input: the static scratch keeps the first call's
contents, which the second must not depend on. A call needing more scratch than
the library holds is refused before any launch.
"""

import dataclasses

import pytest
import torch

from loopspec_amd import _lib, workloads
from tests.conftest import announce

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)

# a bf16 row set with a repetition penalty, then a smaller fp32 one without
FIRST = dataclasses.replace(workloads.C4, name="noalloc-first", batch=8)
SECOND = dataclasses.replace(workloads.C3, name="noalloc-second", batch=4, vocab=8192)


def _args(cfg, inp, drafts, accept_len, tokens):
    t, d = inp["target"], inp["draft"]
    pen = cfg.penalty != 1.0
    h, hl = inp["history"], inp["history_len"]
    return [
        t.data_ptr(), t.stride(0), t.stride(1), d.data_ptr(), d.stride(0), d.stride(1),
        drafts.data_ptr(), inp["uniforms"].data_ptr(), _lib.dtype_code(t), cfg.batch, cfg.k, cfg.vocab,
        float(cfg.temperature), float(cfg.top_p), 0, float(cfg.penalty),
        h.data_ptr() if pen else None, h.stride(0) if pen else 0, hl.data_ptr() if pen else None,
        accept_len.data_ptr(), tokens.data_ptr(),
    ]


def _case(cfg, seed):
    inp = workloads.sampling_inputs(cfg, seed, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed + 17)
    drafts = torch.randint(0, cfg.vocab, (cfg.batch, cfg.k), generator=g, device=DEV, dtype=torch.int64)
    # half the drafts are the target's argmax, so that both accepts and rejects occur
    best = inp["target"][:, : cfg.k].float().argmax(dim=-1)
    drafts[: cfg.batch // 2] = best[: cfg.batch // 2]
    return inp, drafts


def _run(name, cfg, inp, drafts, workspace=None):
    accept_len = torch.full((cfg.batch,), -7, dtype=torch.int32, device=DEV)
    tokens = torch.full((cfg.batch, cfg.k + 1), -7, dtype=torch.int64, device=DEV)
    args = _args(cfg, inp, drafts, accept_len, tokens)
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel()]
    args.append(_lib.stream(DEV))
    _lib.call(name, *args)
    torch.cuda.synchronize()
    return accept_len.cpu(), tokens.cpu()


def test_noalloc_matches_workspace_entry_point_twice():
    cases = [(FIRST, 31), (SECOND, 32)]
    prepared = [(cfg,) + _case(cfg, seed) for cfg, seed in cases]
    # the no-allocation calls back to back, the larger first
    got = []
    for cfg, inp, drafts in prepared:
        announce(f"no_alloc: ls_spec_verify_noalloc {cfg.name} B={cfg.batch} k={cfg.k} V={cfg.vocab}")
        got.append(_run("ls_spec_verify_noalloc", cfg, inp, drafts))
    for (cfg, inp, drafts), (a_na, t_na) in zip(prepared, got):
        nbytes = _lib.query("ls_spec_verify_workspace", cfg.batch, cfg.k, cfg.vocab)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        announce(f"no_alloc: ls_spec_verify {cfg.name}")
        a_ws, t_ws = _run("ls_spec_verify", cfg, inp, drafts, workspace=ws)
        assert torch.equal(a_na, a_ws), cfg.name
        assert torch.equal(t_na, t_ws), cfg.name
        assert (a_na >= 0).all() and (a_na <= cfg.k).all()
        assert 0 < int(a_na.sum()) < cfg.batch * cfg.k  # accepts and rejects both occurred


def test_noalloc_repeat_is_identical():
    cfg = SECOND
    inp, drafts = _case(cfg, 33)
    announce(f"no_alloc: repeat {cfg.name}")
    first = _run("ls_spec_verify_noalloc", cfg, inp, drafts)
    second = _run("ls_spec_verify_noalloc", cfg, inp, drafts)
    assert torch.equal(first[0], second[0]) and torch.equal(first[1], second[1])


def test_noalloc_refuses_calls_above_its_scratch():
    need = _lib.query("ls_spec_verify_workspace", 4096, 8, 262144)
    assert need > 16 << 20
    with pytest.raises(ValueError, match="16 MiB"):
        _lib.call("ls_spec_verify_noalloc", None, 0, 0, None, 0, 0, None, None, 0, 4096, 8, 262144,
                  1.0, 0.9, 0, 1.0, None, 0, None, None, None, None)
