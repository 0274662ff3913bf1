"""Seeded synthetic voxel sets for the benchmark configurations.

All generators return int32 coordinates (N, 4) = (b, x, y, z), unique and
sorted lexicographically (the order voxelisation + ``torch.unique``
produces), built with numpy on the host from a fixed seed.

  config1  B=2, 64^3, 4096 uniform unique voxels (the reference's CPU-sized case)
  config2  B=4, 1440x1440x41 LiDAR-like: a smooth ground heightfield sampled on
           concentric scan rings around a sensor plus ~200 axis-aligned box
           surfaces; ~120k voxels per sample, ~3-8 of 27 neighbours occupied
  config5  B=1, 256^3 indoor-like: random axis-aligned planar walls and floors,
           2 voxels thick; ~1M voxels
"""

import numpy as np

__all__ = ["config1", "config2", "config5", "pack", "unpack", "neighbour_stats"]

_SHIFT = np.array([48, 32, 16, 0], dtype=np.int64)


def pack(c: np.ndarray) -> np.ndarray:
    c = np.asarray(c, dtype=np.int64)
    return (c[:, 0] << 48) | (c[:, 1] << 32) | (c[:, 2] << 16) | c[:, 3]


def unpack(k: np.ndarray) -> np.ndarray:
    return ((k[:, None] >> _SHIFT[None, :]) & 0xFFFF).astype(np.int32)


def _unique(c: np.ndarray) -> np.ndarray:
    return unpack(np.unique(pack(c)))


def config1(seed: int = 0):
    """(coords, spatial_shape): 4096 uniform voxels in 2 x 64^3."""
    rng = np.random.default_rng(seed)
    S = 64
    lin = np.sort(rng.choice(2 * S ** 3, 4096, replace=False))
    c = np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], axis=1).astype(np.int32)
    return c, (S, S, S)


def _heightfield(rng, X, Y, Z):
    ph = rng.uniform(0, 2 * np.pi, 6)
    fx = rng.uniform(60, 160, 3)
    fy = rng.uniform(60, 160, 3)

    def h(x, y):
        v = Z * 0.3 + 2.5 * np.sin(x / fx[0] + ph[0]) + 2.0 * np.sin(y / fy[0] + ph[1])
        v = v + 1.5 * np.sin((x + y) / fx[1] + ph[2]) + 1.0 * np.sin((x - y) / fy[1] + ph[3])
        return np.clip(np.rint(v), 0, Z - 1).astype(np.int64)

    return h


def _lidar_sample(rng, b, X, Y, Z, rings=80, azimuths=2600, boxes=200):
    h = _heightfield(rng, X, Y, Z)
    cx, cy = X / 2 + rng.uniform(-20, 20), Y / 2 + rng.uniform(-20, 20)
    # Scan rings: radii grow geometrically away from the sensor, as the beams of
    # a spinning LiDAR hit the ground at increasing spacing.
    radii = 12.0 * (1.062 ** np.arange(rings))
    radii = radii[radii < min(X, Y) / 2 - 2]
    theta = np.linspace(0, 2 * np.pi, azimuths, endpoint=False)
    rr, tt = np.meshgrid(radii, theta, indexing="ij")
    gx = np.rint(cx + rr * np.cos(tt)).astype(np.int64).ravel()
    gy = np.rint(cy + rr * np.sin(tt)).astype(np.int64).ravel()
    ok = (gx >= 0) & (gx < X) & (gy >= 0) & (gy < Y)
    gx, gy = gx[ok], gy[ok]
    pts = [np.stack([np.full_like(gx, b), gx, gy, h(gx, gy)], axis=1)]
    # Box surfaces (vehicles, walls): the faces seen from the sensor, sampled densely.
    for _ in range(boxes):
        r = rng.uniform(15, min(X, Y) / 2 - 60)
        a = rng.uniform(0, 2 * np.pi)
        x0, y0 = int(cx + r * np.cos(a)), int(cy + r * np.sin(a))
        sx, sy, sz = rng.integers(8, 40), rng.integers(8, 40), rng.integers(4, 14)
        z0 = int(h(np.array([x0]), np.array([y0]))[0])
        xs, ys, zs = np.arange(x0, x0 + sx), np.arange(y0, y0 + sy), np.arange(z0, min(Z, z0 + sz))
        # two faces: x = x0 plane and y = y0 plane
        fy_, fz_ = np.meshgrid(ys, zs, indexing="ij")
        fx_ = np.full_like(fy_, x0)
        gx2, gz2 = np.meshgrid(xs, zs, indexing="ij")
        gy2 = np.full_like(gx2, y0)
        face = np.concatenate([np.stack([fx_.ravel(), fy_.ravel(), fz_.ravel()], 1),
                               np.stack([gx2.ravel(), gy2.ravel(), gz2.ravel()], 1)])
        keep = rng.random(face.shape[0]) < 0.6
        face = face[keep]
        ok = (face[:, 0] >= 0) & (face[:, 0] < X) & (face[:, 1] >= 0) & (face[:, 1] < Y)
        face = face[ok]
        pts.append(np.concatenate([np.full((face.shape[0], 1), b), face], axis=1))
    return np.concatenate(pts).astype(np.int64)


def config2(seed: int = 0, batch: int = 4):
    """(coords, spatial_shape): LiDAR-like scene per sample, B=4, 1440x1440x41."""
    rng = np.random.default_rng(seed)
    X, Y, Z = 1440, 1440, 41
    c = np.concatenate([_lidar_sample(rng, b, X, Y, Z) for b in range(batch)])
    return _unique(c), (X, Y, Z)


def config5(seed: int = 0, target: int = 1_000_000):
    """(coords, spatial_shape): 2-voxel-thick planar walls and floors in 256^3, ~1M voxels."""
    rng = np.random.default_rng(seed)
    S = 256
    keys = np.empty(0, dtype=np.int64)
    while keys.shape[0] < target:
        axis = rng.integers(0, 3)
        pos = rng.integers(0, S - 2)
        lo = rng.integers(0, S // 2, size=2)
        hi = lo + rng.integers(S // 3, S, size=2)
        hi = np.minimum(hi, S)
        u = np.arange(lo[0], hi[0])
        v = np.arange(lo[1], hi[1])
        uu, vv = np.meshgrid(u, v, indexing="ij")
        for t in range(2):
            w = np.full(uu.size, pos + t)
            if axis == 0:
                xyz = np.stack([w, uu.ravel(), vv.ravel()], 1)
            elif axis == 1:
                xyz = np.stack([uu.ravel(), w, vv.ravel()], 1)
            else:
                xyz = np.stack([uu.ravel(), vv.ravel(), w], 1)
            c = np.concatenate([np.zeros((xyz.shape[0], 1), np.int64), xyz], 1)
            keys = np.union1d(keys, pack(c))
    keys = np.sort(rng.permutation(keys)[:target])
    return unpack(keys), (S, S, S)


def neighbour_stats(coords: np.ndarray) -> float:
    """Mean number of occupied sites in each voxel's 3x3x3 neighbourhood (self included)."""
    k = np.sort(pack(coords))
    total = 0
    for dx in (-1, 0, 1):
        for dy in (-1, 0, 1):
            for dz in (-1, 0, 1):
                q = coords.astype(np.int64) + np.array([0, dx, dy, dz])
                ok = (q[:, 1:] >= 0).all(1)
                qk = pack(np.where(ok[:, None], q, 0))
                pos = np.searchsorted(k, qk)
                pos = np.minimum(pos, k.shape[0] - 1)
                total += int(((k[pos] == qk) & ok).sum())
    return total / max(1, coords.shape[0])
