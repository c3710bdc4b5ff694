"""CPU oracle for the LongSpark verify-and-refresh hot path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference's torch
algorithms on the CPU in fp32 (fp64 where a check needs ground truth), op for
op, so that the HIP kernels in ``longspark_amd`` can be checked against it.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or as the timed CPU
baseline.  The product path never routes through this package.

Every function cites the reference file:line it follows.  Where the reference
delegates to a closed binary (sgl-kernel ``top_k_renorm_prob`` /
``top_p_renorm_prob``, flashinfer ``softmax``), the oracle follows the torch
form the reference itself carries (``layers/sampler.py``) and states the tie
rule it adopts; those points are marked "parity unpinned" against the closed
binary and are pinned here by brute force and closed forms instead.

Modules:
  verify   -- greedy verify, acceptance, residual resampling, temperature /
              top-k / top-p / min-p target distributions, penalties, bitmask.
  summary  -- Global16 position scores, online-softmax merge, full-prefix state.
  kvwindow -- Raw256 page table, recent-window gather, ring append.
  draft_attention -- the drafter's attention over the window, summary and
              local views (one-kernel form and merge form).
"""
