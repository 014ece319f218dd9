"""CPU oracle for the compressed-KV decode-attention path. TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it. The GPU path in `insitu_amd` must never call into it (it fails loudly when
its HIP library is missing instead of falling back here).

It restates, in plain numpy (and in C for long contexts, `oracle/c/`), the
reference's fixed-point algorithm. Every function cites the reference file and
line it follows (paths relative to the reference repository root).

How each part is pinned (so a plausible mistake fails a check):

  fixed.rshift/lshift/Q       closed-form tie tables (tests/test_oracle_numerics.py)
  fixed.fwht                  dense Sylvester Hadamard matrix (textbook)
  rotate.*                    tb/vectors rot_signs/rot_random_in/out, rot_q/k/v
  codebook.gaussian(2, 4)     tb/vectors cb_centroids_*/enc_bounds_*
  codebook.gaussian(3)        published Max-Lloyd optimum to 2e-3 and symmetry
                              only -> "parity unpinned" at the integer level
  quantize.*                  tb/vectors enc_in/enc_norm/enc_idx_*, kv_rows,
                              cache_rows_h*; isqrt invariant; brute-force
                              pack/unpack round trips
  layout.DdrLayout            tb/vectors ddr_image.hex + ddr_map.json
  attention.qtab              tb/vectors qtab_table.hex
  attention.scores            tb/vectors scores.hex, score_edge_*; exact
                              Python-int restatement
  attention.ExpLut            tb/vectors exp_table/exp_in/exp_out (every
                              reachable output) and float exp to 1 LSB
  attention.attend_online     tb/vectors sm_*/sm2_* per-token state and
                              out.online.hex end to end
  attention.attend_two_pass   tb/vectors out.hex
  attention.reciprocal/final  tb/vectors fin_*
  c/oracle.c                  equal to the numpy functions above on seeded
                              cases (tests/test_oracle_numerics.py,
                              test_native_oracle_equals_numpy_oracle)
"""
