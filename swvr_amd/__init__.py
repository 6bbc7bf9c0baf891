"""swvr_amd: ``softmax(h @ W.T + b) @ E`` and an MSE loss on it, on MI355X (gfx950).

Drop-in for pengzhangzhi/swvr's public API (swvr/__init__.py:1-6): the same
names, argument shapes, autograd and loss options, computed by hand-written
HIP kernels through the C ABI of include/swvr.h without materialising the
``[N, V]`` scores.
"""
from .api import SoftmaxReadoutMSE, default_chunk_size, softmax_readout, softmax_readout_mse
from .reference import softmax_readout_reference

__all__ = ["softmax_readout", "softmax_readout_mse", "SoftmaxReadoutMSE", "softmax_readout_reference"]
__version__ = "0.1.0"
