"""CPU oracle for the kernel_lab hot path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the original project's
ground truth (kernel_lab/reference.py of Markkoby3/Kernel-lab): fused
residual-add + RMSNorm and paged-KV decode attention, in float32 PyTorch with
the same rounding points, plus an independent float64 NumPy brute force used to
pin it.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the reported CPU
baseline. The product (``kernel-lab_amd/``) never imports it: the operators run
the HIP kernels or raise.

Pinning (each check is in tests/test_oracle.py):

* ``reference.rms_norm``: torch.nn.functional.rms_norm; the unit-RMS invariant;
  a hand-computed closed form; float64 brute force; committed golden vectors.
* ``reference.fused_add_rms_norm``: residual against the correctly rounded
  float64 sum (fp16 and bf16, where double rounding through fp32 is exact);
  normed output as above.
* ``reference.paged_decode_attention``: SDPA on contiguous K/V
  (``dense_decode_attention``); float64 token-loop brute force; the original
  tests' one-hot known answer (13.0); poisoned spare pages; committed golden
  vectors; planted mistakes (GQA mapping, scale, length, page order) that the
  golden vectors must reject.

* ``reference.paged_decode_attention_fp8``: the E4M3 widening against
  ``brute.e4m3_table`` (decoded from the OCP bit layout, all 256 codes); the
  scale identities (k_scale folds into ``scale``, v_scale multiplies the
  output); float64 brute force on the dequantised cache; a one-hot known
  answer in exactly representable E4M3 values.

There are no reference golden files to pin against: the original project's
tests use seeded random data and the known answers above.
"""
