"""MI355X-native weight streaming behind FlexTensor's offload API.

Host logic (planning, scheduling, the offload phases) is Python over PyTorch;
device work goes through the HIP C-ABI library ``libftx_hip.so``
(``include/ftx.h``): pinned host arenas, SDMA / zero-copy-kernel copy
engines, a batched scatter kernel and hipEvent gating.
"""

__version__ = "0.1.0"
