"""SamplingDecisionPolicy drop-in: filter, sample, verify and resolve endpoints.

Same constructor, queue/read/resolve contract, decision packing ([M, 5] int64:
token, proposed, accepted_code, first_rejected, second_rejected) and RNG order
as sglang_recurrent/loopspec/sampling/policy.py:19-308, on this package's
gfx950 sampler. One difference a caller never sees in results: the rejected
q1 rows of a batch are resolved by one batched rejection launch
(RejectionSampler.queue_many) instead of one graph replay per row; it draws the
same two uniforms per row in the same order.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..decisions import DecisionBatch, DecisionOutcome, DecisionReadback
from .distributions import prepare_sampling_probabilities, sample_probabilities


@dataclass
class SamplingDecisionBatch(DecisionBatch):
    verification_distributions: dict | None = None


class SamplingDecisionPolicy:
    """Filter, sample, verify and resolve speculative endpoint logits (policy.py:19-308)."""

    def __init__(self, max_rows, device, options, sampler, *, generator=None):
        if torch.device(device).type != "cuda":
            raise RuntimeError("LoopSpec sampling requires CUDA")
        self.readback = DecisionReadback(max_rows, device)
        self.options = options
        self.sampler = sampler
        self.generator = generator
        self.constants = torch.tensor([0, 1], dtype=torch.int64, device=device)
        self.proposal_token_host = torch.empty(max_rows, dtype=torch.int64, pin_memory=True)
        self.proposal_token_device = torch.empty(max_rows, dtype=torch.int64, device=device)
        self.verification_token_host = torch.empty(max_rows, dtype=torch.int64, pin_memory=True)
        self.verification_token_device = torch.empty(max_rows, dtype=torch.int64, device=device)
        self.sample_row_host = torch.empty(max_rows, dtype=torch.int64, pin_memory=True)
        self.sample_row_device = torch.empty(max_rows, dtype=torch.int64, device=device)
        self.rejection_host = torch.empty((max_rows, 3), dtype=torch.int64, pin_memory=True)
        self.rejection_ready = torch.cuda.Event()
        self.top_p_thresholds = torch.full((max_rows, 1), options["top_p"], dtype=torch.float32, device=device)

    @staticmethod
    def _stage_values(values, host_buffer, device_buffer):
        count = len(values)
        host = host_buffer[:count]
        host.copy_(torch.as_tensor(values, dtype=torch.int64))
        staged = device_buffer[:count]
        staged.copy_(host, non_blocking=True)
        return staged

    def _sample_drafts(self, entries, q1_context, staged_q1_rows):
        """q2 residual proposals first (slot 0), then q1 draws (slot 2) (policy.py:78-142)."""
        proposal_states = {}
        q2_entries = []
        for row, kind, lane, distribution in entries:
            if kind == "q1":
                proposal_states[row] = distribution
            elif kind == "q2":
                q2_entries.append((row, lane, distribution))
        q2_actions = {}
        draft_samples = {}
        if q2_entries:
            q2_targets = torch.stack([d for _, _, d in q2_entries])
            selected = self._stage_values([lane.first_token for _, lane, _ in q2_entries],
                                          self.proposal_token_host, self.proposal_token_device)
            firsts = torch.stack([lane.first_state for _, lane, _ in q2_entries])
            proposals, actions, sampled = self.sampler.sample_conditional_residual(
                firsts, q2_targets, selected, self.generator, result_slot=0)
            for i, (row, _, _) in enumerate(q2_entries):
                proposal_states[row] = proposals[i]
                q2_actions[row] = actions[i]
                draft_samples[row] = sampled[i]
        q1_entries = [row for row, kind, _, _ in entries if kind == "q1"]
        if q1_entries:
            if q1_context is None:
                distributions = torch.stack([d for _, kind, _, d in entries if kind == "q1"])
                samples = sample_probabilities(distributions, self.generator, self.sampler, result_slot=2)
            else:
                samples = self.sampler.sample_top_p(*q1_context, self.generator, result_slot=2,
                                                    sample_rows=staged_q1_rows)
            draft_samples.update({row: samples[i] for i, row in enumerate(q1_entries)})
        return proposal_states, q2_actions, draft_samples

    def _sample_finals(self, entries):
        """Direct final draws (slot 1) and q1 verification decisions (policy.py:144-195)."""
        distributions = {row: d for row, kind, _, d in entries if kind == "final"}
        direct = [(row, d) for row, kind, lane, d in entries if kind == "final" and lane.first_token is None]
        direct_samples = {}
        if direct:
            sampled = sample_probabilities(torch.stack([d for _, d in direct]), self.generator, self.sampler,
                                           result_slot=1)
            direct_samples = {row: sampled[i] for i, (row, _) in enumerate(direct)}
        verification = [(row, lane, d) for row, kind, lane, d in entries
                        if kind == "final" and lane.first_token is not None]
        decisions = {}
        if verification:
            target_masses = torch.stack([d[lane.first_token] for _, lane, d in verification])
            proposal_masses = torch.stack([lane.first_state[lane.first_token] for _, lane, _ in verification])
            tokens = self._stage_values([lane.first_token for _, lane, _ in verification],
                                        self.verification_token_host, self.verification_token_device)
            packed = self.sampler.verify(target_masses, proposal_masses, tokens, self.generator)
            decisions = {row: packed[i] for i, (row, _, _) in enumerate(verification)}
        return distributions, direct_samples, decisions

    def _pack(self, entries, q2_actions, drafts, direct, verification):
        """[M, 5] decisions in endpoint order (policy.py:197-218)."""
        zero, one = self.constants
        none = (zero, zero, zero)
        values = []
        for row, kind, lane, _ in entries:
            if kind == "q1":
                decision = (drafts[row], one, *none)
            elif kind == "q2":
                action = q2_actions[row]
                decision = (torch.where(action > 0, drafts[row], lane.first_token),
                            (action > 0).to(torch.int64), action, zero, zero)
            elif lane.first_token is None:
                decision = (direct[row], zero, *none)
            else:
                decision = verification[row]
            values.extend(decision)
        return torch.stack(values).reshape(-1, 5)

    def queue(self, post_output, endpoints, lanes):
        logits = post_output.next_token_logits
        q1_rows = [row for row, kind in enumerate(endpoints.values()) if kind == "q1"]
        staged_q1_rows = self._stage_values(q1_rows, self.sample_row_host, self.sample_row_device)
        distributions, q1_context = prepare_sampling_probabilities(
            logits, top_p_thresholds=self.top_p_thresholds, sampler=self.sampler, **self.options)
        entries = [(row, kind, lanes[row], d)
                   for (row, kind), d in zip(endpoints.items(), distributions, strict=True)]
        proposal_states, q2_actions, drafts = self._sample_drafts(entries, q1_context, staged_q1_rows)
        verification_distributions, direct, verification = self._sample_finals(entries)
        staged = self.readback.stage(self._pack(entries, q2_actions, drafts, direct, verification))
        return SamplingDecisionBatch(staged, proposal_states=proposal_states,
                                     verification_distributions=verification_distributions)

    def read(self, lanes, endpoints, batch):
        """Host decisions; q1 rejections resolved by the batched fallback (policy.py:255-283)."""
        values = self.readback.read(batch.staged)
        decisions = dict(zip(endpoints, values, strict=True))
        rejected = [(row, d) for row, d in decisions.items() if d[0] < 0]
        if not rejected:
            return decisions
        lanes_r = [lanes[row] for row, _ in rejected]
        self.sampler.rejections.queue_many(
            [lane.first_state for lane in lanes_r],
            [batch.verification_distributions[row] for row, _ in rejected],
            [lane.second_token for lane in lanes_r],
            [lane.second_state for lane in lanes_r],
            self.generator, self.rejection_host)
        self.rejection_ready.record()
        self.rejection_ready.synchronize()
        results = self.rejection_host[: len(rejected)].tolist()
        for (_, decision), (token, second_accepted, second_rejected) in zip(rejected, results, strict=True):
            decision[0] = token
            decision[2] = 2 if second_accepted else 0
            decision[4] = second_rejected
        return decisions

    def resolve(self, lane, endpoint_kind, decision, proposal_state, schedule):
        prediction, proposed, accepted_code, first_rejected, second_rejected = decision
        proposed = bool(proposed)
        if accepted_code == 1:
            accepted_stage = schedule.proposal_stage
        elif accepted_code == 2:
            accepted_stage = schedule.second_stage
        else:
            accepted_stage = None
        return DecisionOutcome(
            prediction=prediction,
            proposed=proposed,
            proposal_state=proposal_state if proposed else None,
            accepted_stage=accepted_stage,
            proposal_action="residual" if endpoint_kind == "q2" and proposed else None,
            first_rejected=bool(first_rejected),
            second_rejected=bool(second_rejected),
        )
