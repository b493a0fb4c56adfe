"""CPU oracle for the packed mixed-precision KV path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the expected result a test compares against (or, for the
baseline, as the timed CPU restatement of the reference's CPU path). The product path (the dkv package and
libdkv.so) never imports it and has no CPU fallback.

Modules:
  kv_quantization  restatement of src/kv_quantization.py (pack/unpack, 64-B header)
  attention        dequantize-then-SDPA oracles (fp64/fp32) and the reference
                   GPU kernel's bf16 rounding semantics (src/gpu_kernels.py:71-105)
  cpu_path         the reference CPU cache flow (src/cache_manager.py:17-90)

Pinning (how each function is checked beyond retyping its formula) is listed in
each module's docstring and tested in tests/test_oracle_*.py.
"""
