"""CPU oracle for the MLX-format affine 4-bit quantized linear path.

TEST INFRASTRUCTURE ONLY.  This package is the checker: tests/, the
``__graft_entry__.smoke()`` check and bench.py's ``cpu_baseline`` leg import
it, nothing else does, and the product library (``aestrix_amd``) never calls
into it -- there is no CPU fallback.

Two restatements of the same algorithm live here:

* ``oracle.ref``   -- numpy, vectorised, used for fixtures and for checks at
  sizes the C version would be slow on in pure Python.
* ``oracle.cref``  -- ctypes binding of ``imq_oracle.c`` (built by the
  ``Makefile`` beside it into ``liboracle.so``), a scalar C loop that follows
  the reference's CPU dequant line by line.

Both follow the reference:

* unpack / affine / RNE: ``Sources/ImarelloDirect/DirectTEEncoder.swift:39-46,106-123``
* y = x . deq(w)^T (transpose=true): ``Sources/ImarelloDirect/DirectQmmSpike.swift:55-58``
* K = packed columns * 8, group size 64, 4 bits:
  ``Sources/ImarelloDirect/DirectDiTStep.swift:853``, ``Sources/ImarelloDiT/TransformerWeights.swift:9-10``

Pinning (which check fixes each function; see tests/test_oracle.py):

* ``f32_to_bf16``: torch's independent RNE conversion on every finite pattern
  class, hand-computed tie cases, overflow to inf.
* ``dequantize``: torch float32 arithmetic + torch RNE (an independent
  implementation) over all 16 codes x a grid of (scale, bias) pairs incl.
  negative, zero and subnormal scales; known-answer words; the special cases
  q=0 -> bf16(bias) and scale=0 -> bias; the C and numpy restatements agree
  bit for bit; planted mutants (high-nibble-first, group k/32, per-op bf16
  rounding) fail.
* ``qmm_t``: torch float64 matmul of the dequantized weight; a rank-1 known
  answer (all codes equal); brute-force pure-Python loops on tiny shapes;
  linearity in x; planted mutants (transposed operand, dropped bias term)
  fail.

The reference's own tests hold no golden vectors for this path (its only
quantization test checks key presence,
``Tests/ImarelloDiTTests/TransformerStructureTests.swift:40-48``), and its
implementation (Swift + MLX + Metal) cannot be built or run here, so there is
no ``oracle/_ref`` build.
"""

from . import ref  # noqa: F401
