"""GPU parity of the greedy kernels against the oracle (bit-exact ids)."""

import numpy as np
import pytest
import torch

from oracle import greedy as og
from loopspec_amd import _lib, verify, workloads
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _oracle(target, draft=None, draft_tokens=None):
    t = target.float().numpy()
    d = None if draft is None else draft.float().numpy()
    dt = None if draft_tokens is None else draft_tokens.numpy()
    return og.greedy_verify(t, d, dt)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_c2_full_shape_bitexact(gpu, seed):
    cfg = workloads.C2
    target, draft = workloads.greedy_inputs(cfg, seed)
    announce(f"greedy C2 seed={seed}")
    rows = torch.empty((cfg.batch, 2 * cfg.k + 1), dtype=torch.int64, device=gpu)
    acc, tok = verify.greedy_verify(target.to(gpu), draft.to(gpu), row_argmax=rows)
    torch.cuda.synchronize()
    a0, t0, r0 = _oracle(target, draft)
    assert np.array_equal(rows.cpu().numpy(), r0)
    assert np.array_equal(acc.cpu().numpy(), a0)
    assert np.array_equal(tok.cpu().numpy(), t0)


@pytest.mark.parametrize("block", [256, 512, 1024])
@pytest.mark.parametrize("splits", [1, 2, 3, 7])
def test_split_counts_agree(gpu, splits, block):
    cfg = workloads.GreedyConfig("t", 8, 3, 49152, torch.bfloat16, tie_frac=0.3)
    target, draft = workloads.greedy_inputs(cfg, 11)
    a0, t0, r0 = _oracle(target, draft)
    _lib.set_option("greedy_splits", splits)
    _lib.set_option("greedy_block", block)
    try:
        for rep in range(3):  # workspace must be left clean for the next call
            announce(f"greedy splits={splits} block={block} rep={rep}")
            rows = torch.empty((8, 7), dtype=torch.int64, device=gpu)
            acc, tok = verify.greedy_verify(target.to(gpu), draft.to(gpu), row_argmax=rows)
            torch.cuda.synchronize()
            assert np.array_equal(rows.cpu().numpy(), r0)
            assert np.array_equal(acc.cpu().numpy(), a0)
            assert np.array_equal(tok.cpu().numpy(), t0)
    finally:
        _lib.set_option("greedy_splits", 0)
        _lib.set_option("greedy_block", 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("vocab", [49152, 1000, 1003])
def test_dtypes_and_unaligned_vocab(gpu, dtype, vocab):
    cfg = workloads.GreedyConfig("t", 5, 2, vocab, dtype, tie_frac=0.5)
    target, draft = workloads.greedy_inputs(cfg, 3)
    announce(f"greedy dtype={dtype} vocab={vocab}")
    acc, tok = verify.greedy_verify(target.to(gpu), draft.to(gpu))
    torch.cuda.synchronize()
    a0, t0, _ = _oracle(target, draft)
    assert np.array_equal(acc.cpu().numpy(), a0)
    assert np.array_equal(tok.cpu().numpy(), t0)


def test_draft_tokens_mode_and_strided_views(gpu):
    cfg = workloads.GreedyConfig("t", 16, 4, 32000, torch.bfloat16)
    target, draft = workloads.greedy_inputs(cfg, 5)
    big = torch.zeros((16, 5, 32008), dtype=torch.bfloat16)
    big[:, :, :32000] = target
    view = big[:, :, :32000]  # row stride 32008 elements
    ids = torch.argmax(draft.float(), dim=-1)
    ids[::3, 0] += 1  # force some first-position rejections
    ids %= 32000
    announce("greedy draft-token mode, strided target")
    acc, tok = verify.greedy_verify(view.to(gpu), draft_tokens=ids.to(gpu))
    torch.cuda.synchronize()
    a0, t0, _ = _oracle(target, draft_tokens=ids)
    assert np.array_equal(acc.cpu().numpy(), a0)
    assert np.array_equal(tok.cpu().numpy(), t0)


def test_special_values(gpu):
    v = 4096
    target = torch.randn((4, 3, v))
    draft = target[:, :2].clone()
    target[0, 0] = -float("inf")  # all -inf -> index 0
    target[1, 0, 17] = float("nan")
    target[1, 0, 900] = float("nan")  # first NaN wins
    target[2, 1] = 0.0
    target[2, 1, 5] = -0.0  # -0 ties +0; lowest index (0) wins
    target[3, 2] = 7.0  # all equal -> 0
    draft[0, 0] = -float("inf")
    announce("greedy special values")
    rows = torch.empty((4, 5), dtype=torch.int64, device=gpu)
    acc, tok = verify.greedy_verify(target.to(gpu), draft.to(gpu), row_argmax=rows)
    torch.cuda.synchronize()
    a0, t0, r0 = _oracle(target, draft)
    assert np.array_equal(rows.cpu().numpy(), r0)
    assert r0[0, 0] == 0 and r0[1, 0] == 17 and r0[2, 1] == 0 and r0[3, 2] == 0
    assert np.array_equal(acc.cpu().numpy(), a0)
    assert np.array_equal(tok.cpu().numpy(), t0)


@pytest.mark.parametrize("rows,vocab", [(1, 49152), (3, 49152), (320, 49152), (7, 128256), (64, 65536)])
def test_argmax_rows(gpu, rows, vocab):
    g = torch.Generator().manual_seed(rows)
    x = (torch.randn((rows, vocab), generator=g) * 3).to(torch.bfloat16)
    announce(f"argmax rows={rows} vocab={vocab}")
    got = verify.argmax_rows(x.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), og.argmax_first(x.float().numpy()))
    got32 = verify.argmax_rows(x.float().to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(got32.cpu().numpy(), torch.argmax(x.float(), -1).numpy())


def test_argmax_rows_inside_graph_replays(gpu):
    """Captured launches replay correctly, each replay checked against eager."""
    x = (torch.randn((6, 49152)) * 3).to(torch.bfloat16).to(gpu)
    out = torch.empty(6, dtype=torch.int64, device=gpu)
    verify.argmax_rows(x, out=out)  # warm up / allocate workspace outside capture
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    announce("argmax graph capture")
    with torch.cuda.graph(graph):
        verify.argmax_rows(x, out=out)
    for rep in range(4):
        out.fill_(-5)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        x[rep, 123] = 100.0  # eager work between replays changes the input
        eager = torch.argmax(x.float(), -1)


@pytest.mark.parametrize("batch,k,vocab,mode", [
    (1, 64, 2048, "logits"),    # the largest k: 129 rows per batch element, the multi-wave combine
    (3, 64, 1000, "tokens"),    # caller draft ids, unaligned vocabulary
    (2, 31, 4096, "logits"),    # 63 rows per element
    (2, 32, 4096, "logits"),    # 65 rows per element
    (5, 1, 4096, "tokens"),     # the smallest k
])
def test_edge_shapes(gpu, batch, k, vocab, mode):
    g = torch.Generator().manual_seed(batch * 1000 + k)
    target = torch.randn(batch, k + 1, vocab, generator=g) * 3
    draft = target[:, :k] + torch.randn(batch, k, vocab, generator=g) * 0.3  # mostly accepted prefixes
    announce(f"greedy edge B={batch} k={k} V={vocab} {mode}")
    if mode == "logits":
        acc, tok = verify.greedy_verify(target.to(gpu), draft.to(gpu))
        a0, t0, _ = _oracle(target, draft)
    else:
        ids = torch.argmax(draft, dim=-1)
        acc, tok = verify.greedy_verify(target.to(gpu), draft_tokens=ids.to(gpu))
        a0, t0, _ = _oracle(target, draft_tokens=ids)
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy(), a0)
    assert np.array_equal(tok.cpu().numpy(), t0)


def test_empty_batch(gpu):
    target = torch.zeros(0, 3, 4096, device=gpu)
    draft = torch.zeros(0, 2, 4096, device=gpu)
    acc, tok = verify.greedy_verify(target, draft)
    torch.cuda.synchronize()
    assert acc.shape == (0,) and tok.shape == (0, 3)


def test_status_word_clear_after_runs_and_reported_when_set(gpu):
    """The workspace's sticky status stays clear over ordinary launches; a
    planted bit is reported by check_greedy_status and cleared by it."""
    target, draft = workloads.greedy_inputs(workloads.C2, 0)
    verify.greedy_verify(target.to(gpu), draft.to(gpu))
    verify.check_greedy_status(gpu)
    ws = _lib.WORKSPACE.get(torch.device(gpu), 0, "greedy")
    word = verify.greedy_status_word(ws)
    assert word is not None and int(word.item()) == 0
    word.fill_(1)
    with pytest.raises(RuntimeError, match="poll limit"):
        verify.check_greedy_status(gpu, ws)
    assert int(word.item()) == 0
    verify.check_greedy_status(gpu, ws)


def test_stream_read_probe_reads_every_word_once(gpu):
    """The read-ceiling kernel's outputs combine to the exclusive-or of every
    word of the target and draft rows (each word is read exactly once)."""
    cfg = workloads.GreedyConfig("probe", 64, 2, 49152, torch.bfloat16)
    target, draft = workloads.greedy_inputs(cfg, seed=4, device=gpu)
    announce("stream_read_probe C2 shape")
    out = verify.stream_read_probe(target, draft)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    words = np.concatenate([target.contiguous().view(torch.int32).cpu().numpy().ravel(),
                            draft.contiguous().view(torch.int32).cpu().numpy().ravel()]).view(np.uint32)
    assert got == np.bitwise_xor.reduce(words)
