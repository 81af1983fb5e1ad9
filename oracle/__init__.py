"""TEST INFRASTRUCTURE ONLY: CPU parity oracle for the sparse-attention hot path.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import
this package, and only as the checker (or the timed CPU baseline), never as the product
path.  The product (``sinkattn_amd``) never imports it.

Contents
--------
torch_ref   CPU torch restatements of the reference functions, each citing the
            reference file:line it follows (exact block mass, max-pool closed form,
            mean-pooled scores, coverage mask, required mask, dense masked softmax
            attention with LSE, LSE mixing, the compensation branch's K/V mean pooling).
c_ref       ctypes loader of oracle/_build/liboracle.so: the plain-C coverage-mask
            restatement (ATen fp32 sum order, fp64 cumsum, libstdc++ std::sort
            emulation) and the real libstdc++ std::sort.

How each function is pinned (tests/test_oracle_*.py):
  exact block mass     fp64 brute force on small shapes; closed forms (rows sum to 1,
                       Q = 0 gives |kb|/N, a dominant sink key gives block 0 -> 1)
  max-pool             the reference kernel's own outputs (tests/golden/max_pool.npz, its
                       Triton source run by Triton's CPU interpreter in float16): bit for
                       bit on inputs whose q.k are exact in fp32, and each of the four
                       rounding points, left out, breaks them; fp64 evaluation of the
                       formula; row normalisation invariant
  mean-pooled scores   closed form (softmax of pooled dot products, padding rule)
  coverage mask        C model vs torch on this machine (sum order, cumsum, sort
                       permutation incl. ties), emulated vs real std::sort, brute-force
                       minimal-k definition on small rows, invariants and special cases
  dense attention      SDPA on a full mask, block-local attention on a diagonal mask,
                       logsumexp identity
  LSE mixing           equals attention over the union of both key sets with the pooled
                       keys counted sample_gap times (fp64 identity); plain average at
                       gap 1 and equal LSEs
  K/V mean pooling     ramp and constant closed forms, replicate-padded last group,
                       prefix rows untouched, identities at gap 1 / prefix >= N
Not pinned by a reference output: the max-pool map in bf16 (Triton's interpreter mishandles
bf16, so the fixtures are float16; bf16 differs only in the rounding format, checked to be
round-to-nearest-even), and its ragged-N behaviour (undefined in the reference).
"""
