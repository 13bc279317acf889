"""MI355X-native (gfx950) continuous-batching hot path of tokserve.

Hand-written HIP kernels (libtokserve_hip.so, C ABI in include/tokserve_hip.h)
for KV append, block-table gathers, paged attention (decode and chunked
prefill), RMSNorm, RoPE and greedy selection, behind Python operators that keep
tokserve's kernel signatures and add packed ragged-batch entry points.
Importing the package does not load the HIP library; the first kernel call does.
"""

__version__ = "0.1.0"
