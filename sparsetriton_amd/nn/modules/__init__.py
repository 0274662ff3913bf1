from .conv import SparseConv3D, SparseConv3DBase, SparseConvTransposed3D, SubMConv3D

__all__ = ["SparseConv3DBase", "SparseConv3D", "SubMConv3D", "SparseConvTransposed3D"]
