from .resnet import SparseResNet, SparseResNet21D

__all__ = ["SparseResNet", "SparseResNet21D"]
