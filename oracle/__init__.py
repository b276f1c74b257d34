"""CPU oracle for the FemtoVLLM attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference for results (or, for
``sdpa_path``, as the timed CPU baseline).  The shipped operators never call
into it; they fail loudly when the HIP library is missing.

* ``attention`` -- float64 numpy restatement (decode, chunked prefill, dense,
  cache write), the primary checker.
* ``sdpa_path`` -- torch-CPU restatement of the reference's own PyTorch
  attention path (femtovllm/models/qwen/qwen3.py:389-544).
* ``brute`` -- pure-Python loops for tiny inputs.

The reference implementation itself cannot be built here: its kernels are a
CUDA torch extension (setup.py:51-90, nvcc) and Triton kernels that need an
NVIDIA GPU, so there is no ``oracle/_ref``.
"""
