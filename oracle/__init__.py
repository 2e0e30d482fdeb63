"""CPU oracle for torch.js's autograd hot path.  TEST INFRASTRUCTURE ONLY.

A numpy restatement of the contract every hot-path op of torch.js
declares (its `@pytorch` tags, e.g. src/tensor/Tensor.ts:4,
src/nn/functional.ts:4, src/optim/adamw.ts:4), following the reference's
own forward formulas where they are well defined (A&S 7.1.26 erf in GELU,
max-subtracted log-softmax, biased-variance LayerNorm, Adam/AdamW update
order, integer-exponent pow, first-max argmax, wrapping gather, ...).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker / the timed CPU baseline.
The 'hip' product path never calls into it.

Every function is pinned by tests/test_oracle.py: golden vectors from
PyTorch in float64, the reference's literal tests, closed forms, special
states of the generator, published known answers and finite differences.
What no check can fix is the reference's own float32 ULP behaviour in the
browser's WGSL built-ins (exp, log, cos, ...), which is implementation-
defined; the oracle evaluates in float64 and the GPU tests compare at the
stated tolerances.

Precision: floating-point work runs in float64 unless a function says it
emulates the reference's float32 rounding (the Adam/AdamW moments).

Modules
  ops    per-op forward / backward (each cites the reference file:line)
  rng    torch.js's seeded LCG + xorshift32 generator
  models GPT-2 / transformer-block / MLP / CNN forward + explicit backward
"""
