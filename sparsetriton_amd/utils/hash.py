"""Coordinate hash table on the GPU, plus the coordinate packing helpers.

Same public surface as the reference (``sparsetriton/utils/hash.py:22-580``):
``HashTable(capacity=None, device="cpu", table_keys=None, table_values=None)``
with ``insert``, ``query``, ``capacity``, ``device``, ``to``, ``cpu`` and the
public ``table_keys`` / ``table_values`` arrays, and the ``flatten_coord`` /
``unflatten_coord`` / ``hash_coords`` helpers.

What differs, by design:

* ``table_keys`` holds exact packed 64-bit coordinates (int64, the layout of
  ``flatten_coord``), not a 31-bit hash of them.  The reference's stored key
  (``hash_coords_kernel2``, ``hash.py:136-152``) aliases distinct coordinates,
  so its table can return a wrong row; this one cannot.
* Probing is bounded by the table size instead of 128 steps, so an insert
  only fails when the table is full; failures are counted in ``status`` and
  ``check()`` raises on them instead of dropping the coordinate.
* Duplicate coordinates resolve to the lowest row index, on every run.
* ``insert`` records the rows; the insert kernel runs when the table arrays
  are first needed (``table_keys`` / ``table_values``, ``query``,
  ``counters``, moving devices).  A submanifold kernel map is built from its
  own brick index (``st_kmap_subm``) and never needs the table.

Insert and query run as HIP kernels (``st_hash_insert`` / ``st_hash_query``);
there is no CPU implementation of them.
"""

import ctypes

import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.config import get_coords_dtype

__all__ = ["HashTable", "StatusSnapshot", "flatten_coord", "hash_coords", "unflatten_coord"]


class StatusSnapshot:
    """Host copy of a device status buffer (``ST_STATUS_WORDS`` int32), taken without stalling
    the stream: the copy into pinned memory is queued behind the kernels that fill the buffer,
    and ``values()`` waits only for that copy -- not for whatever the stream runs after it."""

    def __init__(self, status: torch.Tensor):
        self._host = torch.empty(tuple(status.shape), dtype=status.dtype, pin_memory=True)
        self._host.copy_(status, non_blocking=True)
        self._event = torch.cuda.Event()
        self._event.record(torch.cuda.current_stream(status.device))
        self._values = None

    def values(self) -> list:
        if self._values is None:
            self._event.synchronize()
            self._values = self._host.tolist()
        return self._values

    def counters(self) -> dict:
        v = self.values()
        return {"overflow": v[_lib.STATUS_OVERFLOW], "bad_coord": v[_lib.STATUS_BAD_COORD],
                "duplicate": v[_lib.STATUS_DUPLICATE], "out_of_box": v[_lib.STATUS_OUT_OF_BOX]}

    def raise_errors(self, capacity: int) -> None:
        """Raise on a full table or coordinates that cannot be keyed (rows the kernels could not
        place: their neighbours would silently be missing)."""
        c = self.counters()
        if c["overflow"]:
            raise RuntimeError(f"HashTable: {c['overflow']} inserts found the table full (capacity {capacity})")
        if c["bad_coord"]:
            raise RuntimeError(
                f"{c['bad_coord']} coordinates outside the packable range "
                "(batch in [0, 32767], x/y/z in [-32768, 32767])"
            )


def flatten_coord(coords: torch.Tensor) -> torch.Tensor:
    """Pack (N, 4) rows (b, x, y, z) into int64 ``b<<48 | x<<32 | y<<16 | z`` (``hash.py:25-54``)."""
    c = coords.to(torch.int64)
    return (c[:, 0] << 48) | ((c[:, 1] & 0xFFFF) << 32) | ((c[:, 2] & 0xFFFF) << 16) | (c[:, 3] & 0xFFFF)


def unflatten_coord(flat_coords: torch.Tensor) -> torch.Tensor:
    """Inverse of ``flatten_coord``; returns (N, 4) in the configured coordinate dtype (``hash.py:57-83``)."""
    f = flat_coords.to(torch.int64)
    parts = [(f >> 48) & 0xFFFF, (f >> 32) & 0xFFFF, (f >> 16) & 0xFFFF, f & 0xFFFF]
    return torch.stack(parts, dim=1).to(get_coords_dtype())


def hash_coords(coords: torch.Tensor) -> torch.Tensor:
    """Non-negative int32 spatial hash of (N, 4) coordinates.

    The reference's host-side helper (``hash.py:86-113``): prime multipliers
    per component, XOR-combined with int32 wrap-around, top bit cleared.  It
    is not used by the table, which keys on exact coordinates.
    """
    c = coords.to(torch.int64)
    h = (c[:, 1] * 73856093) ^ (c[:, 2] * 19349663) ^ (c[:, 3] * 83492791) ^ (c[:, 0] * 1000003)
    return (h & 0x7FFFFFFF).to(torch.int32)


class HashTable:
    """Open-addressing table mapping packed coordinates to row indices.

    ``table_keys`` (int64, -1 = empty) and ``table_values`` (int32, -1 =
    none) have ``capacity`` slots each.  Build with ``insert`` (rows get their
    index in the inserted tensor), look up with ``query`` (-1 when absent).
    """

    def __init__(self, capacity: int = None, device="cpu", table_keys: torch.Tensor = None,
                 table_values: torch.Tensor = None):
        assert capacity is not None or (table_keys is not None and table_values is not None), (
            "Either capacity or both table_keys and table_values must be provided."
        )
        self._pending = None  # (coords, scale) recorded by insert(), applied by _materialize()
        self._needs_clear = False
        self.status = None
        self._build_ws = None  # zeroed workspace of st_hash_build (left zeroed by every build)
        if table_keys is not None and table_values is not None:
            assert table_keys.shape == table_values.shape, "table_keys and table_values must have the same shape."
            self._keys, self._vals = table_keys, table_values
        else:
            capacity = int(capacity)
            assert capacity > 0, "capacity must be positive"
            device = torch.device(device)
            self._keys = torch.empty((capacity,), dtype=torch.int64, device=device)
            self._vals = torch.empty((capacity,), dtype=torch.int32, device=device)
            self.clear()

    # ------------------------------------------------------------ properties
    @property
    def table_keys(self) -> torch.Tensor:
        self._materialize()
        return self._keys

    @table_keys.setter
    def table_keys(self, value: torch.Tensor) -> None:
        self._materialize()
        self._keys = value

    @property
    def table_values(self) -> torch.Tensor:
        self._materialize()
        return self._vals

    @table_values.setter
    def table_values(self, value: torch.Tensor) -> None:
        self._materialize()
        self._vals = value

    @property
    def device(self) -> torch.device:
        return self._keys.device

    @device.setter
    def device(self, device) -> None:
        self._materialize()
        self._keys = self._keys.to(device, non_blocking=True)
        self._vals = self._vals.to(device, non_blocking=True)
        if self.status is not None:
            self.status = self.status.to(device, non_blocking=True)

    def cpu(self) -> "HashTable":
        self.device = torch.device("cpu")
        return self

    def to(self, device) -> "HashTable":
        self.device = device
        return self

    @property
    def capacity(self) -> int:
        return self._keys.shape[0]

    # ------------------------------------------------------------ operations
    def clear(self) -> "HashTable":
        """Mark every slot empty (keys and values all-ones, i.e. -1)."""
        self._pending = None
        if self._keys.is_cuda:
            self._needs_clear = True  # filled when the table is next needed
        else:
            self._keys.fill_(-1)
            self._vals.fill_(-1)
        return self

    def _materialize(self) -> None:
        """Apply the deferred clear and insert: a clear followed by an insert is one partitioned
        build into the table as empty (``st_hash_build``, no fill); the CAS insert
        (``st_hash_insert``) after a fill where that build is not available."""
        if self._pending is not None:
            keys, scale = self._pending
            self._pending = None
            fresh = self._needs_clear
            self._needs_clear = False
            if self._build(keys, scale, fresh):
                return
            if fresh:
                _lib.fill_(self._keys, -1)
                _lib.fill_(self._vals, -1)
            _lib.call("st_hash_insert", _lib.ptr(keys), _lib.coord_code(keys.dtype), keys.shape[0], int(scale),
                      _lib.ptr(self._keys), _lib.ptr(self._vals), self.capacity,
                      _lib.ptr(self._status()), _lib.stream_of(self.device))
        elif self._needs_clear:
            self._needs_clear = False
            _lib.fill_(self._keys, -1)
            _lib.fill_(self._vals, -1)

    def _build(self, keys: torch.Tensor, scale: int, fresh: bool) -> bool:
        """``st_hash_build`` of ``keys`` into the table; False when the table is too large for it or
        the 16-lane probe mode is on (the caller then runs the CAS insert)."""
        lib = _lib.lib()
        n = keys.shape[0]
        nbytes = ctypes.c_int64()
        rc = lib.st_hash_build_workspace(n, self.capacity, ctypes.byref(nbytes))
        if rc == _lib.ERR_UNSUPPORTED:
            return False
        _lib.check(rc, "st_hash_build_workspace")
        if self._build_ws is None or self._build_ws.numel() < nbytes.value or self._build_ws.device != self.device:
            self._build_ws = torch.zeros((nbytes.value,), dtype=torch.uint8, device=self.device)
        rc = lib.st_hash_build(_lib.ptr(keys), _lib.coord_code(keys.dtype), n, int(scale), _lib.ptr(self._keys),
                               _lib.ptr(self._vals), self.capacity, 1 if fresh else 0, _lib.ptr(self._build_ws),
                               self._build_ws.numel(), _lib.ptr(self._status()), _lib.stream_of(self.device))
        if rc == _lib.ERR_UNSUPPORTED:
            return False
        _lib.check(rc, "st_hash_build")
        return True

    def _status(self) -> torch.Tensor:
        if self.status is None or self.status.device != self.device:
            self.status = torch.zeros(_lib.STATUS_WORDS, dtype=torch.int32, device=self.device)
        return self.status

    def insert(self, keys: torch.Tensor, scale: int = 1) -> None:
        """Insert (N, 4) coordinate rows; row i is stored with value i.

        ``scale`` multiplies x, y, z before packing (the transposed-conv table
        over ``coords * stride``).  Asynchronous: call ``check()`` to surface
        a full table or unpackable coordinates.
        """
        keys = keys.contiguous()
        n = keys.shape[0]
        assert self.capacity >= n, (
            "Hash table capacity should be at least twice the number of keys to ensure low collision rate."
        )
        assert keys.ndim == 2 and keys.shape[1] == 4, "keys must have shape (N, 4)"
        _lib.require_device(self._keys, "HashTable")
        if keys.device != self.device:
            keys = keys.to(self.device)
        assert self._keys.dtype == torch.int64 and self._vals.dtype == torch.int32, (
            "HashTable arrays must be int64 keys / int32 values"
        )
        _lib.coord_code(keys.dtype)  # rejects unsupported coordinate dtypes now
        if self._pending is not None:
            self._materialize()  # an earlier pending insert goes first (the clear stays deferred otherwise)
        self._pending = (keys, int(scale))

    def query(self, keys: torch.Tensor) -> torch.Tensor:
        """Row index of each (N, 4) coordinate, or -1 when absent (int32, shape (N,))."""
        keys = keys.contiguous()
        n = keys.shape[0]
        _lib.require_device(self.table_keys, "HashTable")
        if keys.device != self.device:
            keys = keys.to(self.device)
        out = torch.empty((n,), dtype=torch.int32, device=self.device)
        _lib.call("st_hash_query", _lib.ptr(keys), _lib.coord_code(keys.dtype), n, _lib.ptr(self.table_keys),
                  _lib.ptr(self.table_values), self.capacity, _lib.ptr(out), _lib.stream_of(self.device))
        return out

    def status_tensor(self) -> torch.Tensor:
        """The device status words the table's kernels count into (``ST_STATUS_WORDS`` int32):
        overflow, bad_coord, duplicate and out_of_box (rows of a submanifold map query outside
        its bounds)."""
        return self._status()

    def snapshot(self) -> StatusSnapshot:
        """Asynchronous host copy of the status words as of the work queued so far (the deferred
        insert is not forced: a table used only through its rank index never runs it)."""
        return StatusSnapshot(self._status())

    def counters(self) -> dict:
        """Device failure counters (synchronises): overflow, bad_coord, duplicate, out_of_box."""
        self._materialize()
        return self.snapshot().counters()

    def check(self) -> None:
        """Raise if any insert found the table full or a coordinate unpackable."""
        self._materialize()
        self.snapshot().raise_errors(self.capacity)
