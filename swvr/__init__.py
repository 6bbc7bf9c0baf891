"""``import swvr`` resolves to swvr_amd, so code written against pengzhangzhi/swvr runs unchanged."""
from swvr_amd import (SoftmaxReadoutMSE, __version__, softmax_readout, softmax_readout_mse,
                      softmax_readout_reference)

__all__ = ["softmax_readout", "softmax_readout_mse", "SoftmaxReadoutMSE", "softmax_readout_reference"]
