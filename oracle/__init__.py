"""CPU oracle of the speculative-decoding hot path -- TEST INFRASTRUCTURE.

A restatement, in PyTorch on the CPU, of the reference algorithms this
repository accelerates (beriltatli/speculative-decoder): spec/accept.py,
lm/sampling.py, spec/ngram.py, cache/paged.py, cache/kv.py, lm/forward.py
(cached Llama forward with the gather copy and SDPA), spec/draft.py,
spec/verify.py, spec/loop.py and baselines/cached_autoregressive.py.  Each
function cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the CPU baseline; the
product path (speculative-decoder_amd/) never does.

How each part is pinned (see tests/test_oracle_*.py): the reference's own
known-answer literals (accept toy fractions, the coupled 120x120 grid,
n-gram and paging literals), golden vectors written by the reference itself
(tests/golden/), brute force on tiny inputs, closed forms, and transformers'
own uncached Llama forward for the model math.
"""
