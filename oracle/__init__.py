"""CPU oracle for the GPT token loop — TEST INFRASTRUCTURE ONLY.

This package restates NimbleML's CPU path (NumPy + nimbleml_native) for the
per-token GPT forward, ``generate`` and ``compute_loss``. It is the checker the
HIP path is compared against. Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
or the timed CPU baseline; the ``nimbleml_amd`` product never imports it.

Modules:
  weights   seeded parameter generator with the reference's npz names
            (NimbleML/utils/saveload.py:16-41).
  gpt_ref   the forward / sampling / generate / loss restatement; each function
            cites the reference file:line it follows.

Pinning (how each oracle function is checked, see tests/test_oracle.py):
  - every function against fixtures written by the real reference
    (tests/golden/make_golden.py imports /root/reference in the build
    container with its native extension compiled into oracle/_ref/);
  - GELU against the reference's compiled gelu_forward (oracle/_ref);
  - RMSNorm, GELU, softmax attention and cross-entropy against float64 closed
    forms; sampling against numpy.random.choice; KV-cache decode against the
    full re-forward.
"""
