"""CPU oracle for the quantized conv path: TEST INFRASTRUCTURE, not product code.

``oracle.reference`` restates FlashIM's torch reference functions (flashim/ops/conv.py, ops/gemm.py, ops/quantize.py,
quant/formats/*.py, quant/tensor.py) in torch on the CPU. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker or the timed CPU baseline. The pinning of each function
(known answers from FlashIM's tests, closed forms, brute force) lives in tests/test_oracle.py. FlashIM's reference is
Python: there is no C reference to build into oracle/_ref.
"""
