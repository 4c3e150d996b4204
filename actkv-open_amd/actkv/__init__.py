"""ActKV eviction hot path for AMD Instinct MI355X (gfx950).

Modules mirror the reference package layout: actkv.kernels.lse_attn (LSE-recovery scoring),
actkv.kernels.compaction (conflict-free in-place compaction) and actkv.paged (PagedKVCache with
keep_mask_from_scores / compact / evict).  Importing the package loads nothing heavy; the HIP
library is loaded on first use.
"""
__version__ = "0.1.0"
