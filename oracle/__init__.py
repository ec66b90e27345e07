"""CPU oracle for the BDH strict-tril attention hot path.

TEST INFRASTRUCTURE ONLY.  This package is the checker, never the product.
Nothing in ``bdh-gpu-fast_amd/`` (the HIP library or its Python surface)
imports, links or calls it.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may use it: as the reference the HIP
results are compared against, and as the timed CPU baseline.

The oracle is a numpy restatement of the reference's CPU path for this op:

* ``csrc/tril_attn_cpu.cpp`` (eager / tiled strict-tril score x V and decode,
  with the same tile pickers and score budgets),
* ``kernels/attention_bwd.py`` (analytic dense and blocked backward,
  merged self-attention gradient),
* ``bdh.py`` / ``kernels/rope.py`` (RoPE frequencies, phases, cos/sin, pair
  rotation incl. the bf16 mixed-precision rounding order, rotation backward).

Every function cites the reference file:line it restates.  How each one is
pinned (golden vectors from the reference's own tests, closed forms, brute
force, invariants) is listed in ``PINNING`` in ``tril_attn_oracle.py`` and
checked by ``tests/test_oracle.py``.
"""

from .tril_attn_oracle import *  # noqa: F401,F403
from .tril_attn_oracle import __all__  # noqa: F401
