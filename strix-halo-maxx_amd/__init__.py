"""MI355X-native (gfx950) hot path of strix-halo-maxx: the moondream2 SigLIP vision tower, the moondream2 text decoder
(prefill + batch-1 greedy decode) and the TAPNext TRecViT block with its RG-LRU recurrence.

Host code is Python on PyTorch-ROCm (device memory and streams only); every hot op is a hand-written HIP kernel in
csrc/ reached through the C ABI of libshmaxx.so (include/shmaxx.h). Import this package as `strix_halo_maxx_amd`.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
