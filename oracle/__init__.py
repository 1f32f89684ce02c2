"""The oracle: a CPU restatement of the reference's paged-KV store / gather
and of its model-runner metadata packing.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import or run anything under oracle/, and
only to check results (or as the timed CPU baseline), never as the thing measured
or shipped.  The product (nano-vllm-multimodal_amd/) never imports it and
fails loudly when its HIP library is missing.

  oracle.paged_kv   numpy / plain-Python restatement (readable form)
  oracle.c_oracle   ctypes wrapper of oracle/nkv_oracle.c (OpenMP C form,
                    fast enough for full-size checks and the CPU baseline)
  oracle.build      gcc recipe for oracle/_build/libnkv_oracle.so

The reference's own native path (csrc/paged_kv) needs the CUDA toolkit and
cannot be compiled here, so there is no oracle/_ref build; how every oracle
function is pinned is listed in tests/test_oracle.py.
"""
