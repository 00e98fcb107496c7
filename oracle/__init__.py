"""CPU oracle for the 12-bit lossless bf16 decode-linear path.

TEST INFRASTRUCTURE ONLY.  Only the test suite (tests/), the smoke check in
__graft_entry__.smoke() and the CPU-baseline leg of bench.py may import, call,
link or execute anything under oracle/, and only as the checker.  The product
path (ai_amd) never routes through this package.

Contents
  codec.py   numpy restatement of compress / decompress
             (ramvi/engine/ramvi_engine/kernels/wcomp.py:13-45)
  linear.py  closed forms of the fused linears gemvc1 / gemvc_tc in float64
             (wcomp.py:57-126, 143-242) and the tensor/order conventions of the
             engine call sites (ramvi/engine/ramvi_engine/core/engine.py:329-356)
  qwen3.py   float32 Qwen3 forward for greedy-token parity
             (ramvi/engine/ramvi_engine/core/reference.py:24-61)
  c/         C restatement of the codec and of the fp32 GEMV / 12-bit
             decode+GEMV used as the timed CPU baseline
             (ramvi/engine/ramvi_engine/cpu/cpu_layer.py:35-48)

Pinning: every function is checked in tests/test_oracle.py against the golden
vectors in tests/golden/codec_golden.npz (written by the reference's own
compress/decompress), the exhaustive bf16 round trip, and closed-form special
cases of the linear (identity rows, single exceptions, brute force).
"""
