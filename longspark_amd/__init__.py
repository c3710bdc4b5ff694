"""MI355X-native LongSpark verify-and-refresh hot path.

Drop-in replacements for the reference's per-round verify (greedy and
rejection-sampling acceptance with penalties, masks, temperature, top-k,
top-p and min-p) and drafter-view refresh (recent-window KV gather, ring
append, summary score/merge), each backed by hand-written gfx950 HIP kernels
in ``liblongspark_amd.so`` behind the C ABI of ``include/longspark_amd.h``.

Importing a submodule that launches kernels loads the library and fails
loudly if it has not been built (``python -m longspark_amd.build``).
"""

__version__ = "0.1.0"
