"""MI355X-native offloaded Qwen3-MoE verification path.

``specfit_amd.runtime`` holds the drop-in Python API (router module, expert
operator, GPU expert cache); ``specfit_amd.ops`` the tensor wrappers of the
C-ABI kernels in ``lib/libspecfit_amd.so`` (built from ``csrc/`` by
``python -m specfit_amd.build``).
"""
__version__ = "0.1.0"
