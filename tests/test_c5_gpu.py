"""The full C5 step on the GPU: C3-shaped speculative verify at B=128, then the
paged commit of each row's accepted tokens' KV (24 layers x 4 loops x {K, V}
= 192 planes of 16 heads x 128 bf16 = 4 KiB token rows, pages of 16, context
lengths U(512, 8192)).

Accept lengths and tokens must equal the oracle's; the commit's destination
slots, page table, context lengths and ring state must equal
oracle.graph_ops.kv_commit_plan's bit for bit, and on sampled planes every
accepted token's row must have moved from its branch slot to its destination
while every other slot is left alone.
"""

import numpy as np
import pytest
import torch

from oracle import graph_ops as og
from oracle import sampling as osmp
from loopspec_amd import verify, workloads
from loopspec_amd.loopspec import graph_ops as go
from tests.conftest import announce

pytestmark = pytest.mark.gpu

SAMPLED_PLANES = (0, 97, 191)


@pytest.mark.parametrize("seed", [11])
def test_c5_full_step(gpu, seed):
    cfg, kvc = workloads.C5_SAMPLING, workloads.C5_KV
    assert (cfg.batch, cfg.k, kvc.planes, kvc.token_bytes, kvc.page_size) == (128, 2, 192, 4096, 16)
    inp = workloads.sampling_inputs(cfg, seed)
    # drafts from the filtered draft distributions (oracle)
    drafts = np.zeros((cfg.batch, cfg.k), dtype=np.int64)
    for b in range(cfg.batch):
        for i in range(cfg.k):
            q = osmp.filter_row(osmp.process_logits(inp["draft"][b, i].numpy(), cfg.temperature), cfg.top_p).P
            drafts[b, i] = osmp.categorical_pick(q, float(inp["draft_uniforms"][b, i]))
    drafts = torch.from_numpy(drafts)
    announce(f"C5 verify B={cfg.batch} seed={seed}")
    acc, tok = verify.speculative_verify(inp["target"].to(gpu), inp["draft"].to(gpu), drafts.to(gpu),
                                         inp["uniforms"].to(gpu), cfg.temperature, cfg.top_p)
    torch.cuda.synchronize()
    want = osmp.speculative_verify(inp["target"].numpy(), inp["draft"].numpy(), drafts.numpy(),
                                   inp["uniforms"].numpy(), cfg.temperature, cfg.top_p)
    assert np.array_equal(acc.cpu().numpy(), want.accept_len)
    assert np.array_equal(tok.cpu().numpy(), want.tokens)
    assert 0 < int(want.accept_len.sum()) < cfg.batch * cfg.k

    state = workloads.kv_commit_state(kvc, cfg.batch, cfg.k, steps=1, seed=seed, device=gpu)
    kv = state["kv"]
    g = torch.Generator(device=gpu).manual_seed(seed)
    for p in range(kv.shape[0]):
        kv[p].copy_(torch.randn(kv[p].shape, generator=g, device=gpu).to(kv.dtype))
    before = {p: kv[p].view(torch.int16).cpu().numpy() for p in SAMPLED_PLANES}
    host = {n: state[n].cpu().numpy() for n in ("page_table", "ctx_len", "free_pages", "page_state", "branch_slots")}
    # the ring as a server holds it: a bounded free run from the cursor
    page_state = torch.tensor([0, len(host["free_pages"])], dtype=torch.int64, device=gpu)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    announce("C5 commit_kv 192 planes")
    dst = go.commit_kv(kv, acc, state["branch_slots"], state["page_table"], state["ctx_len"], state["free_pages"],
                       page_state, kvc.page_size, status=status)
    torch.cuda.synchronize()
    wdst, wpt, wcl, wstate, wstatus = og.kv_commit_plan(
        want.accept_len, host["branch_slots"], host["page_table"], host["ctx_len"], host["free_pages"],
        (0, len(host["free_pages"])), kvc.page_size, state["num_pages"])
    assert wstatus == 0 and status.item() == 0
    assert np.array_equal(dst.cpu().numpy(), wdst)
    assert np.array_equal(state["page_table"].cpu().numpy(), wpt)
    assert np.array_equal(state["ctx_len"].cpu().numpy(), wcl)
    assert tuple(page_state.cpu().tolist()) == wstate
    assert (wcl - host["ctx_len"] == want.accept_len).all()
    branch = host["branch_slots"]
    for p in SAMPLED_PLANES:
        after = kv[p].view(torch.int16).cpu().numpy()
        expect = og.kv_commit_copy(before[p][None].copy(), branch, wdst)[0]
        assert np.array_equal(after, expect), p
