"""Seeded synthetic inputs for the benchmark configurations.

All inputs are generated with torch on the requested device from an explicit
seed, so a CPU copy of a GPU input (or a CPU-generated input copied to the GPU)
is the common ground for parity checks. Shapes follow the configurations of
the verify-and-sample benchmark:

- C1: greedy, B=1, k=2, V=49152, fp32 (CPU baseline shape)
- C2: greedy, B=64, k=2, V=49152, bf16, 1% planted argmax ties
- C3: sampling, B=64, k=2, V=49152, fp32, T=1.0, top_p=0.7
- C4: sampling, B=32, k=4, V=128256, bf16, T=0.7, top_p=0.9, repetition 1.1
- C5: C3 at B=128 followed by the paged KV commit
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class GreedyConfig:
    name: str
    batch: int
    k: int
    vocab: int
    dtype: torch.dtype
    tie_frac: float = 0.0
    target_std: float = 3.0
    noise_std: float = 1.0


C1 = GreedyConfig("C1-greedy-b1-k2-v49152-fp32", 1, 2, 49152, torch.float32)
C2 = GreedyConfig("C2-greedy-b64-k2-v49152-bf16", 64, 2, 49152, torch.bfloat16, tie_frac=0.01)


def greedy_inputs(cfg: GreedyConfig, seed: int, device: torch.device | str = "cpu"):
    """Return (target [B,k+1,V], draft [B,k,V]) logits in cfg.dtype.

    Final-loop logits ~ N(0, target_std^2); draft = final + N(0, noise_std^2)
    at the first k positions. A fraction tie_frac of all B*(2k+1) rows gets
    an exact copy of its maximum planted at another, uniformly chosen index,
    so lowest-index tie-breaking is exercised.
    """
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    b, k, v = cfg.batch, cfg.k, cfg.vocab
    target = torch.randn((b, k + 1, v), generator=g, device=device) * cfg.target_std
    draft = target[:, :k] + torch.randn((b, k, v), generator=g, device=device) * cfg.noise_std
    target = target.to(cfg.dtype)
    draft = draft.to(cfg.dtype)
    if cfg.tie_frac > 0:
        rows = torch.cat([target.reshape(b * (k + 1), v), draft.reshape(b * k, v)])
        n = rows.shape[0]
        pick = torch.rand(n, generator=g, device=device) < cfg.tie_frac
        idx = torch.nonzero(pick).flatten()
        if idx.numel():
            maxv, argm = rows[idx].float().max(dim=-1)
            other = torch.randint(0, v, (idx.numel(),), generator=g, device=device)
            other = torch.where(other == argm, (other + 1) % v, other)
            rows[idx, other] = maxv.to(cfg.dtype)
            target = rows[: b * (k + 1)].reshape(b, k + 1, v).contiguous()
            draft = rows[b * (k + 1):].reshape(b, k, v).contiguous()
    return target.contiguous(), draft.contiguous()


def greedy_algorithmic_bytes(cfg: GreedyConfig, with_draft_logits: bool = True) -> int:
    """Bytes a greedy step must move at least once: every logit read once."""
    elem = torch.tensor([], dtype=cfg.dtype).element_size()
    rows = cfg.batch * (cfg.k + 1) + (cfg.batch * cfg.k if with_draft_logits else 0)
    out = cfg.batch * 4 + cfg.batch * (cfg.k + 1) * 8
    return rows * cfg.vocab * elem + out
