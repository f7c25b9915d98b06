"""CPU oracle for the QuIP# quantize/dequantize hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``: results are compared against it, or it is timed as the CPU baseline.
The product package ``quipsharp_amd`` never imports anything from here.

Two restatements of numbersletter/quipsharp live here:

* ``qs_oracle.c`` (loaded through :mod:`oracle.cref`) -- scalar fp32 C, one IEEE
  operation at a time, for the integer/bit-level parts: E8P and E8 1-bit tables,
  encode, decode, residual VQ and the Walsh-Hadamard transform.
* :mod:`oracle.torch_path` -- a torch-CPU restatement of the layer pipeline
  (incoherence, BlockLDLQ, quantize_linear, dense-dequantize linear_forward)
  with the reference's own tensor shapes, used to time the reference CPU cost
  and to check end-to-end behaviour within tolerance.
"""
