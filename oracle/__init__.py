"""CPU oracle for the quantized DiT linear path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the reference's eager
PyTorch semantics for the W8A8 / W4A8 linear path so that the HIP kernels can be
checked against it. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker (or as
the timed CPU baseline). The product package ``mx_qlinear`` never imports it and
has no CPU fallback.

Modules
-------
``bf16``        bit-exact bfloat16 / float16 rounding helpers (numpy).
``eager_np``    numpy restatement of each function on the path (quantizer, exact
                int32 GEMM, dequant epilogue, W4 pack/decode, grouped W4A8, adaLN,
                tanh-GELU), each citing the reference lines it follows.
``eager_torch`` torch-CPU restatement of the reference's eager op sequence
                (``torch._int_mm`` + chunked dequant). It is the CPU baseline that
                ``bench.py`` times and a second, independent restatement that the
                tests cross-check against ``eager_np``.

Pinning status of each function (what checks it besides a restatement):
  quantize_int8_rowwise   KATs (constant / zero / one-hot / tie rows), brute-force
                          agreement with eager_torch, row-slice invariance.
  int8_matmul             int64 brute force, identity / permutation weights.
  dequant_epilogue        closed forms with power-of-two scales, eager_torch.
  gelu_tanh_bf16          exhaustive 65,536-entry table from torch CPU (golden
                          fixture); torch is the routine the reference calls.
  adaln                   float64 LayerNorm bound + bf16 op KATs; eager_torch.
  dequant_int4_grouped_to_int8  closed form over all 16 codes x power-of-two
                          scales; s_rel = 1 gives c - 8 exactly.
  w4a8_grouped_linear     per-group int64 brute force; float64 combination. The
                          group-128 fp16-scale format has no reference
                          implementation: parity unpinned by the reference.
"""

from . import bf16, eager_np  # noqa: F401
