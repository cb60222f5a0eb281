from .spiking_resnet import SpikingBottleneck, SpikingResNet, fold_bn_, spiking_resnet50

__all__ = ["SpikingBottleneck", "SpikingResNet", "fold_bn_", "spiking_resnet50"]
