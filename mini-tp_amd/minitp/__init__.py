"""minitp on MI355X: mini-tp's TP=1 Qwen2 token loop on hand-written HIP kernels.

The public modules mirror the reference package layout (``minitp.config``,
``minitp.parallel.linear``, ``minitp.kv_cache``, ``minitp.generation`` ...)
so code written against mini-tp imports unchanged. Compute runs only in
libminitp.so on a ROCm device; there is no CPU path.
"""

__version__ = "0.4.0+mi355x"
