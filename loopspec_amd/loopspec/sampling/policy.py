"""SamplingDecisionPolicy drop-in (interface of
sglang_recurrent/loopspec/sampling/policy.py:19-308: constructor, queue / read /
resolve, the [M, 5] decision rows (token, proposed, accepted_code,
first_rejected, second_rejected) and the generator's draw order).

One cycle is one device buffer and one round trip. Every endpoint's decision
row is written into `decisions` [max_rows, 5] on the device by the sampler's
kernels and a few index writes; queue() ends with one copy of the used rows
to pinned host memory and read() waits once. A verified row's residual
fallback (after a rejected q1 proposal) runs in the same cycle: the rejection
kernel takes every verified row and its result is kept where the row was
rejected, so there is no second round trip.

Draw order, as the reference consumes the generator: q2 residual proposals,
q1 draws, direct final draws, the verify draws, then two uniforms per rejected
row in row order. Those last pairs are drawn ahead, one torch.rand(2) per
verified row: the r-th rejected row takes the r-th pair, the pair the
reference's r-th fallback draws. read(), knowing the number of rejections,
sets the generator's offset to where it stands after that many pairs.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..decisions import DecisionBatch, DecisionOutcome
from .distributions import prepare_sampling_probabilities, sample_probabilities

# decision row columns
TOKEN, PROPOSED, ACCEPTED, FIRST_REJ, SECOND_REJ = range(5)


@dataclass
class SamplingDecisionBatch(DecisionBatch):
    verification_distributions: dict | None = None
    # verified rows (positions) and the generator offsets of their drawn-ahead pairs
    verified: tuple = ()
    pair_offsets: tuple = ()


class SamplingDecisionPolicy:
    """Filter, sample, verify and resolve speculative endpoint logits."""

    def __init__(self, max_rows, device, options, sampler, *, generator=None):
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("LoopSpec sampling requires CUDA")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        self.max_rows = max_rows
        self.options = options
        self.sampler = sampler
        self.generator = generator
        self.decisions = torch.zeros((max_rows, 5), dtype=torch.int64, device=device)
        self.decisions_host = torch.empty((max_rows, 5), dtype=torch.int64, pin_memory=True)
        self.ready = torch.cuda.Event()
        # the cycle's integers, staged with one copy: 4 index lists and 3 token lists
        self.ints_host = torch.empty(7 * max_rows, dtype=torch.int64, pin_memory=True)
        self.ints = torch.empty(7 * max_rows, dtype=torch.int64, device=device)
        self.pairs = torch.empty((max_rows, 2), dtype=torch.float32, device=device)
        self.no_second = torch.zeros(sampler.vocabulary_size, dtype=torch.float32, device=device)
        self.top_p_thresholds = torch.full((max_rows, 1), options["top_p"], dtype=torch.float32, device=device)

    def _generator(self) -> torch.Generator:
        return self.generator if self.generator is not None else torch.cuda.default_generators[self.device.index]

    def _stage(self, lists):
        """One pinned copy of several int lists; returns their device views."""
        flat = [v for values in lists for v in values]
        if not flat:
            return [self.ints[:0] for _ in lists]
        n = len(flat)
        self.ints_host[:n].copy_(torch.tensor(flat, dtype=torch.int64))
        self.ints[:n].copy_(self.ints_host[:n], non_blocking=True)
        views, at = [], 0
        for values in lists:
            views.append(self.ints[at:at + len(values)])
            at += len(values)
        return views

    def queue(self, post_output, endpoints, lanes):
        logits = post_output.next_token_logits
        rows = list(endpoints)
        kinds = list(endpoints.values())
        m = len(rows)
        if m > self.max_rows:
            raise ValueError(f"{m} endpoint rows exceed max_rows {self.max_rows}")
        lane_of = [lanes[r] for r in rows]
        q1 = [i for i, k in enumerate(kinds) if k == "q1"]
        q2 = [i for i, k in enumerate(kinds) if k == "q2"]
        direct = [i for i, k in enumerate(kinds) if k == "final" and lane_of[i].first_token is None]
        verified = [i for i, k in enumerate(kinds) if k == "final" and lane_of[i].first_token is not None]
        q1_d, q2_d, direct_d, ver_d, q2_tok, ver_tok, ver_meta = self._stage([
            q1, q2, direct, verified,
            [lane_of[i].first_token for i in q2],
            [lane_of[i].first_token for i in verified],
            [v for i in verified for v in (lane_of[i].second_token or 0, int(lane_of[i].second_state is not None))],
        ])
        distributions, q1_context = prepare_sampling_probabilities(
            logits, top_p_thresholds=self.top_p_thresholds, sampler=self.sampler, **self.options)
        gen = self.generator
        dec = self.decisions[:m]
        dec.zero_()
        proposal_states = {rows[i]: distributions[i] for i in q1}

        if q2:
            firsts = torch.stack([lane_of[i].first_state for i in q2])
            proposals, actions, drawn = self.sampler.sample_conditional_residual(
                firsts, distributions.index_select(0, q2_d), q2_tok, gen, result_slot=0)
            took = actions > 0
            dec[q2_d, TOKEN] = torch.where(took, drawn, q2_tok)
            dec[q2_d, PROPOSED] = took.to(torch.int64)
            dec[q2_d, ACCEPTED] = actions.to(torch.int64)
            proposal_states.update({rows[i]: proposals[j] for j, i in enumerate(q2)})

        if q1:
            if q1_context is None:
                drawn = sample_probabilities(distributions.index_select(0, q1_d), gen, self.sampler,
                                             result_slot=2)
            else:
                drawn = self.sampler.sample_top_p(*q1_context, gen, result_slot=2, sample_rows=q1_d)
            dec[q1_d, TOKEN] = drawn
            dec[q1_d, PROPOSED] = 1

        if direct:
            dec[direct_d, TOKEN] = sample_probabilities(distributions.index_select(0, direct_d), gen,
                                                        self.sampler, result_slot=1)

        pair_offsets = ()
        if verified:
            n = len(verified)
            firsts = torch.stack([lane_of[i].first_state for i in verified]).float()
            targets = distributions.index_select(0, ver_d)
            at = torch.arange(n, device=self.device)
            packed = self.sampler.verify(targets[at, ver_tok], firsts[at, ver_tok], ver_tok, gen)
            # the fallback pairs, one per verified row, in draw order
            g = self._generator()
            offsets = [g.get_offset()]
            for r in range(n):
                torch.rand(2, out=self.pairs[r], generator=gen)
                offsets.append(g.get_offset())
            pair_offsets = tuple(offsets)
            rejected = packed[:, 0] < 0
            rank = torch.cumsum(rejected.to(torch.int64), 0) - rejected.to(torch.int64)
            seconds = torch.stack([lane_of[i].second_state if lane_of[i].second_state is not None
                                   else self.no_second for i in verified]).float()
            fallback = torch.empty((n, 3), dtype=torch.int64, device=self.device)
            self.sampler.rejections._launch(firsts, targets, seconds, ver_meta.view(n, 2),
                                            self.pairs[:n].index_select(0, rank), fallback, n)
            dec[ver_d] = packed
            dec[ver_d, TOKEN] = torch.where(rejected, fallback[:, 0], packed[:, 0])
            dec[ver_d, ACCEPTED] = torch.where(rejected, 2 * fallback[:, 1], packed[:, 2])
            dec[ver_d, SECOND_REJ] = torch.where(rejected, fallback[:, 2], packed[:, 4])

        self.decisions_host[:m].copy_(dec, non_blocking=True)
        self.ready.record()
        return SamplingDecisionBatch(
            (m, 5), proposal_states=proposal_states,
            verification_distributions={rows[i]: distributions[i] for i, k in enumerate(kinds) if k == "final"},
            verified=tuple(verified), pair_offsets=pair_offsets)

    def read(self, lanes, endpoints, batch):
        """The cycle's decisions after one wait; the generator is left where the
        reference's would be after its fallback draws."""
        del lanes
        m, _ = batch.staged
        self.ready.synchronize()
        values = self.decisions_host[:m].tolist()
        if batch.verified:
            rejections = sum(values[i][FIRST_REJ] for i in batch.verified)
            self._generator().set_offset(batch.pair_offsets[rejections])
        return dict(zip(endpoints, values, strict=True))

    def resolve(self, lane, endpoint_kind, decision, proposal_state, schedule):
        """DecisionOutcome of one decision row (policy.py:285-308)."""
        del lane
        token, proposed, code = decision[TOKEN], bool(decision[PROPOSED]), decision[ACCEPTED]
        stage = {1: schedule.proposal_stage, 2: schedule.second_stage}.get(code)
        return DecisionOutcome(
            prediction=token,
            proposed=proposed,
            proposal_state=proposal_state if proposed else None,
            accepted_stage=stage,
            proposal_action="residual" if proposed and endpoint_kind == "q2" else None,
            first_rejected=bool(decision[FIRST_REJ]),
            second_rejected=bool(decision[SECOND_REJ]),
        )
