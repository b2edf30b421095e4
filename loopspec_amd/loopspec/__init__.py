"""Drop-in mirror of the reference's ``sglang_recurrent.loopspec`` hot path.

Same module names, call signatures, argument meanings and error types as the
reference's sampler, distributions, rejection, policies, decisions and graph
ops; every device computation runs in the gfx950 kernels of
libloopspec_hip.so through the C-ABI. There is no CPU fallback: a missing
library raises at first use.
"""
