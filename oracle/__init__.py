"""CPU oracle for the SignRound v2 tuning path -- TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference's algorithm, written from the reference
files cited in each function (``mround/reference/*.py``, ``mround/core/*.py``,
``mround/formats/*.py``, ``mround/planner/sensitivity.py``). It exists to check
the HIP path, nothing else: only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it, and there only as the
checker or the timed CPU baseline. The ``mround_amd`` package never imports it
and has no CPU fallback.

Every function takes a ``dtype``. With ``np.float32`` the arithmetic is the
reference's float32 arithmetic operation for operation (IEEE division, round
half to even, the reference's order of operations), which is what the GPU
kernels are held to bit for bit on codes and reconstructions. With
``np.float64`` it is the reference's NumPy oracle (``mround/reference``).

Pinning (what checks each part beyond restating its formula):

* ``quantize``: the reference's hand-computed cases, sign convention and
  clamp-boundary fixture, and central finite differences of the explicit
  straight-through surrogate for every branch (tests/test_oracle_quantize.py).
* ``optimizer``: exact step size, sign(0), loss-scale invariance, schedule end
  and total excursion (tests/test_oracle_optimizer.py).
* ``losses``: the reference's global-selection value, denominator and k >= 1
  rules, threshold-versus-exact-k semantics, finite differences.
* ``packing``: the 0x76543210 known answer, bit positions and straddlers, and
  an independent explode-and-reassemble construction.
* ``sensitivity``: the reference's hand values (0.9 and 2.0), storage costs.
* ``block``: a float64 PyTorch-CPU decoder block, cross-checked against the
  Hugging Face ``Qwen2DecoderLayer``/``LlamaDecoderLayer`` and by finite
  differences.
"""
