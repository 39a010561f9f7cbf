"""CPU oracle for the quantized-GEMM operator path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the math of the reference PyTorch modules that define each op
(the ``Model.forward`` of the kernelbench-harbor task families; every function cites the
reference file:line it follows). It is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it. The
product path (``kernelbench_harbor_amd``) never imports, calls or falls back to it.

Pinning (what keeps each function honest, beyond re-typing the formula). Every op also has
committed golden vectors under tests/golden/ (torch's CPU library routines running the reference
modules' op sequences on small seeded inputs; the reference itself ships none):
  numerics      fp16 / bf16 rounding checked against torch's CPU casts (library routines);
                e4m3fn decode table exhaustively against torch.float8_e4m3fn; e4m3fn RNE
                encoder exhaustively on all fp16 inputs against torch; e8m0 closed form KATs.
  w4a16         unpack KATs (0x76543210, 0xFEDCBA98, 0x80000000), pack/unpack inverse,
                one-hot identity GEMM, brute-force dequant loops on tiny shapes, committed
                golden vectors (tests/golden).
  w8a8          int32 accumulate KATs (all +127 -> 231225344, alternating signs, -128), brute
                force int64 loops, closed-form epilogue order.
  fp8w          decode table + brute force; block scale index k // BLOCK checked with one-hot
                scale rows (the reference oracle's k0 // 32 mistake fails this check).
  mxfp8         scale = 2^ceil(log2(amax/448)) KATs, dequant round trip |q*scale - x| bounds,
                exact power-of-two GEMM KAT.
  qmoe          top-2 closed form w1 = 1/(1+exp(l2-l1)), dense-vs-sparse equivalence on tiny
                shapes, brute-force loops.
  qmoe_ffn      golden vectors from a torch per-token loop (fp32 ground truth and the fused
                fp16 sequence with h, expert outputs and combine rounded); float64
                per-token loops written from the definition on tiny shapes (32-row groups);
                a closed form (one-hot x, up weights dequantising to 1, one down row of 3s)
                whose output is 3 * silu(gate) combined, bit-exact in fp16, which fails if
                gate and up trade places; silu against torch.nn.functional.silu.
  silu_fp8      golden vectors (torch CPU ops of the reference sequence); silu(x) = x exactly
                for x >= 17 (e^-x < 2^-24), so act is exact there; the group's absmax element
                quantises to +-448; power-of-two scales make act/scale exact, so crafted values
                on and between e4m3 grid points (ties) pin the RNE codes; |out - act| within
                half an e4m3 step of each group.
"""
