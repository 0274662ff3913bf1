from .tile import mask_spatial_range

__all__ = ["mask_spatial_range"]
