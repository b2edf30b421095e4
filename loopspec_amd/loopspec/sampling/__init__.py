"""Sampling drop-ins: CategoricalSampler, RejectionSampler, distributions, policy."""
