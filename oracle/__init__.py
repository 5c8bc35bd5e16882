"""CPU oracle for the KeSSie hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's own algorithm for the path
the GPU library implements, one function per reference function, each citing
the reference file:line it follows:

  oracle.fog        fog V-weights and fog logit bias  (kessie_hip_kernels.py:403-413,
                    kessie_attention.py:114-139)
  oracle.attention  windowed / fused-fog attention and its paged + GQA decode
                    and chunked-prefill forms  (kessie_hip_kernels.py:577-593)
  oracle.rope       RoPE remap and its frequency table  (kessie_hip_kernels.py:596-606)
  oracle.pages      page insert / threshold evict / free-list order / gather
                    order  (kessie_kernels_v2.hip:393-456, kessie_hip_kernels.py:484-570)
                    and the score-eviction / compaction rule built on them

Who may use it: ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` -- and only as the reference the results
are compared with (or the timed CPU baseline), never as the thing measured or
shipped.  The product package
``kessie_amd`` never imports it.

How it is pinned (tests/test_oracle_*.py): the reference ships no golden
vectors for this path, so each function is checked against the known answers
the reference's own tests assert (page-evict count 64, fog-bias closed forms,
RoPE identity / round trip), against closed forms and special cases the
mathematics fixes (full RoPE composition, single-key and constant-V
attention, GQA = per-head attention, window >= N = full), and against brute
force on tiny inputs.  Functions without such a check say "parity unpinned"
in their docstring.
"""
