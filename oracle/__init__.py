"""CPU oracle for the fused-group path — TEST INFRASTRUCTURE, NOT PRODUCT.

A NumPy restatement of the reference's ``ReferenceExecutor`` and
``runtime/ops.py`` (mdlc/runtime/reference.py:41-199, mdlc/runtime/ops.py:
1-255), making the same NumPy calls (``np.einsum("ok,nkp->nop")`` for conv,
``a @ b`` for gemm) so its results are the reference's results. It also
defines the INT8 quantized semantics the reference never built (``quant``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline. The ``mdlc_amd`` product never imports it.

How each function is pinned (besides restating the reference) is listed in
``tests/test_oracle.py``: closed forms, torch CPU float64 convolution and
pooling, brute-force loops on tiny inputs, and exact integer arithmetic.
"""

from oracle.reference import ReferenceExecutor, run_reference  # noqa: F401
