"""MI355X-native LoopSpec verify-and-sample path.

Hand-written gfx950 HIP kernels behind a C-ABI (include/loopspec_hip.h), with
Python drop-ins that keep the call signatures of the reference's
``sglang_recurrent.loopspec`` sampler, verifier and graph ops:

- ``loopspec_amd.loopspec``: drop-in mirror of the reference modules
  (decisions, sampling.sampler/distributions/rejection/policy, graph_ops).
- ``loopspec_amd.verify``: batched fused entry points (greedy and speculative
  chain verification, KV-timeline commit).
"""

from . import _lib

__all__ = ["_lib"]
