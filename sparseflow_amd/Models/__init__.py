from .spiking_resnet import (SpikingBottleneck, SpikingResNet, calibrate_lif_thresholds_, fold_bn_, fuse_conv_lif_,
                             spiking_resnet50)
from .spikformer import (SPS, SSA, Spikformer, SpikformerBlock, SpikingMLP, spikformer_cifar_4_384,
                         spikformer_cifar_small, spikformer_cifar_tiny)

__all__ = ["SpikingBottleneck", "SpikingResNet", "calibrate_lif_thresholds_", "fold_bn_", "fuse_conv_lif_", "spiking_resnet50", "SPS", "SSA", "Spikformer",
           "SpikformerBlock", "SpikingMLP", "spikformer_cifar_4_384", "spikformer_cifar_small",
           "spikformer_cifar_tiny"]
