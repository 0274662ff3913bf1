"""SparseTensor: features (N, C) on active voxels with coordinates (N, 4) = (b, x, y, z).

Same constructor, properties and methods as the reference
(``sparsetriton/tensor.py:27-457``): ``feats``/``F``, ``coords``/``C`` (cast
to the configured coordinate dtype on the features' device),
``spatial_shape`` (max + 1 when not given), ``batch_size``, ``to``, ``cpu``,
``half``, ``float``, ``dense``, ``replace`` (shares the cache), ``+`` and
``randn``.

``TensorCache`` carries what the convolution path builds once per coordinate
set and reuses across layers: the coordinate hash table and, per convolution
geometry ``(kernel, stride, padding, dilation, submanifold, transposed)``, the
output coordinates, kernel map and output shape (``conv.py:143-191``).
"""

from typing import Any, Dict, List, Optional, Tuple, Union

import torch

from sparsetriton_amd.config import get_coords_dtype
from sparsetriton_amd.utils.hash import HashTable
from sparsetriton_amd.utils.to_dense import to_dense

__all__ = ["SparseTensor", "TensorCache", "randn"]


class TensorCache:
    """Per-coordinate-set cache shared by a tensor and its ``replace()`` descendants."""

    def __init__(self) -> None:
        self.kmaps: Dict[Tuple[Any, ...], Any] = {}
        self.hashtable: Optional[HashTable] = None
        self.neighbor_indices: Dict[Tuple[Any, ...], Tuple[torch.Tensor, Any, Tuple]] = {}


class SparseTensor:
    """Sparse 3-D tensor: ``feats`` (N, C) at ``coords`` (N, 4) = (batch, x, y, z)."""

    def __init__(
        self,
        feats: torch.Tensor,
        coords: torch.Tensor,
        spatial_shape: Optional[Tuple[int, ...]] = None,
        batch_size: Optional[int] = None,
        cache: Optional[TensorCache] = None,
    ) -> None:
        self.feats = feats
        self.coords = coords.to(device=feats.device, dtype=get_coords_dtype())

        assert self.feats.shape[0] == self.coords.shape[0], "The number of features and coordinates must match."
        assert self.coords.shape[1] == 4, "Coordinates must have shape (N, 4)."
        assert self.feats.ndim == 2 and self.coords.ndim == 2, "Features and coordinates must be 2D tensors."

        if spatial_shape is None:
            if self.coords.shape[0] > 0:
                self.spatial_shape = torch.Size((self.coords[:, 1:].max(dim=0).values + 1).tolist())
            else:
                self.spatial_shape = torch.Size([0, 0, 0])
        else:
            if isinstance(spatial_shape, torch.Tensor):
                spatial_shape = spatial_shape.tolist()
            self.spatial_shape = torch.Size([int(s) for s in spatial_shape])

        if batch_size is None:
            self.batch_size = int(self.coords[:, 0].max().item() + 1) if self.coords.shape[0] > 0 else 0
        else:
            if self.coords.shape[0] > 0:
                max_b = self.coords[:, 0].max().item()
                assert batch_size > max_b, f"batch_size {batch_size} must be > max batch index {max_b}"
            self.batch_size = batch_size

        self._cache = TensorCache() if cache is None else cache

    # ------------------------------------------------------------ accessors
    @property
    def F(self) -> torch.Tensor:
        return self.feats

    @F.setter
    def F(self, feats: torch.Tensor) -> None:
        self.feats = feats

    @property
    def C(self) -> torch.Tensor:
        return self.coords

    @C.setter
    def C(self, coords: torch.Tensor) -> None:
        self.coords = coords.to(get_coords_dtype())

    # ------------------------------------------------------------ conversions
    def to(self, device: Union[str, torch.device], non_blocking: bool = False) -> "SparseTensor":
        self.feats = self.feats.to(device, non_blocking=non_blocking)
        self.coords = self.coords.to(device, non_blocking=non_blocking)
        return self

    def cpu(self) -> "SparseTensor":
        return self.to("cpu")

    def half(self) -> "SparseTensor":
        self.feats = self.feats.half()
        return self

    def float(self) -> "SparseTensor":
        self.feats = self.feats.float()
        return self

    def dense(self) -> torch.Tensor:
        """Channels-last dense tensor (B, X, Y, Z, C)."""
        return to_dense(self.feats, self.coords, self.spatial_shape)

    def replace(self, feats: torch.Tensor) -> "SparseTensor":
        """Same coordinates, shape, batch size and cache with new features.

        The coordinates were validated when this tensor was built, so no
        device reduction (and no host synchronisation) happens here.
        """
        assert feats.ndim == 2 and feats.shape[0] == self.coords.shape[0], "The number of features and coordinates must match."
        out = SparseTensor.__new__(SparseTensor)
        out.feats = feats
        out.coords = self.coords if self.coords.device == feats.device else self.coords.to(feats.device)
        out.spatial_shape = self.spatial_shape
        out.batch_size = self.batch_size
        out._cache = self._cache
        return out

    def __repr__(self) -> str:
        return (
            f"SparseTensor(\n"
            f"  feats=tensor(shape={self.feats.shape}, dtype={self.feats.dtype}, device={self.feats.device}),\n"
            f"  coords=tensor(shape={self.coords.shape}, dtype={self.coords.dtype}, device={self.coords.device}),\n"
            f"  spatial_shape={self.spatial_shape}\n"
            f")"
        )

    def __add__(self, other: Union["SparseTensor", torch.Tensor]) -> "SparseTensor":
        if isinstance(other, SparseTensor):
            # Residual connection: both operands share the coordinate set.
            return self.replace(self.feats + other.feats)
        raise NotImplementedError("Addition with dense tensors not yet supported")


def randn(
    spatial_shape: Tuple[int, ...],
    batch_size: int = 1,
    channels: int = 1,
    nnz: int = 100,
    device: Union[str, torch.device] = "cpu",
    dtype: torch.dtype = torch.float32,
) -> SparseTensor:
    """Random SparseTensor with ``nnz`` unique coordinates and N(0, 1) features.

    Coordinates come out lexicographically sorted (b, x, y, z), as the
    reference's ``torch.unique``-based sampler produces (``tensor.py:381-457``).
    """
    total = batch_size * spatial_shape[0] * spatial_shape[1] * spatial_shape[2]
    if nnz > total:
        raise ValueError(f"nnz ({nnz}) exceeds total available voxels ({total})")

    c_dtype = get_coords_dtype()
    pool: List[torch.Tensor] = []
    have = 0
    while have < nnz:
        need = nnz - have
        draw = int(need * 1.2) if have > 0 else nnz
        cols = [torch.randint(0, batch_size, (draw, 1), device=device, dtype=c_dtype)]
        for dim in spatial_shape:
            cols.append(torch.randint(0, dim, (draw, 1), device=device, dtype=c_dtype))
        fresh = torch.cat(cols, dim=1)
        merged = torch.cat([pool[0], fresh], dim=0) if pool else fresh
        pool = [torch.unique(merged, dim=0)]
        have = pool[0].shape[0]

    coords = pool[0][:nnz].contiguous()
    feats = torch.randn(nnz, channels, device=device, dtype=dtype, requires_grad=True).contiguous()
    return SparseTensor(feats, coords, spatial_shape=spatial_shape)
