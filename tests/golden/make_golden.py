"""Writes the golden fixtures under tests/golden/.

reference_kats.json
    Known-answer vectors transcribed from the reference's own tests and
    docstrings (data only; each entry names its source file:line).
conv_cases.npz
    Small sparse-convolution cases in the shapes of the reference's
    tests/test_sparse_conv.py parametrisations (10^3 grid, nnz 27 / 100 / 120),
    with expected values from dense torch.nn.functional.conv3d /
    conv_transpose3d in float64 on the CPU -- the same independent library
    routine the reference's tests compare against (test_sparse_conv.py:37-44,
    69-76, 109-122, 150-156):
      out_coords  set of reachable output sites (nonzero of the dense
                  convolution of the occupancy grid with an all-ones kernel),
                  sorted lexicographically
      out         dense output read at out_coords
      dX, dW      gradients of sum(out * dY) w.r.t. the input features and the
                  (k^3, C_in, C_out) weight, by dense autograd
    Inputs are float32-representable; expected values are computed in float64
    and stored as float32.

Run: python tests/golden/make_golden.py
"""

import json
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent

KATS = {
    "flatten_coord": {
        "source": "tests/test_utils_hash.py:12-32",
        "cases": [
            {"coords": [[0, 1, 2, 3]], "flat": [(0 << 48) | (1 << 32) | (2 << 16) | 3]},
            {"coords": [[1, 255, 255, 255]], "flat": [(1 << 48) | (255 << 32) | (255 << 16) | 255]},
        ],
        "roundtrip": [[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3], [1, 100, 200, 50]],
    },
    "hash_table": {
        "source": "tests/test_utils_hash.py:95-123; sparsetriton/utils/hash.py:379-391, 555-564",
        "cases": [
            {"insert": [[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3]], "capacity": 1000,
             "query": [[0, 1, 2, 3], [0, 1, 2, 4]], "expect": [0, 1]},
            {"insert": [[0, 1, 2, 3]], "capacity": 1000, "query": [[0, 5, 5, 5]], "expect": [-1]},
            {"insert": [[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3], [1, 0, 0, 0]], "capacity": 1000,
             "query": [[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3], [1, 0, 0, 0]], "expect": [0, 1, 2, 3]},
            {"insert": [[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3]], "capacity": 1000,
             "query": [[0, 1, 2, 3], [0, 1, 2, 4], [0, 5, 5, 5]], "expect": [0, 1, -1]},
        ],
    },
    "offset_convention": {
        "source": "tests/test_correctness_vs_spconv.py:44-59; sparsetriton/nn/functional/conv/kmap.py:122-131",
        "note": "k = (dx + K//2) * K^2 + (dy + K//2) * K + (dz + K//2) for base offset (dx, dy, dz)",
        "kernel_size": 3,
        "base_offsets_shape": [27, 3],
        "k_of": {"-1,-1,-1": 0, "0,0,0": 13, "1,1,1": 26, "-1,0,1": 5, "1,0,-1": 21},
    },
    "reference_hash_alias": {
        "source": "sparsetriton/utils/hash.py:116-152 (closed forms)",
        "note": "key2 of (0,0,0,0) and (1,10,0,29) is 0 for both: the reference's stored key aliases",
        "a": [0, 0, 0, 0],
        "b": [1, 10, 0, 29],
        "key2": 0,
        "h1_b": 17432605,
    },
    "build_out_coords_docstring": {
        "source": "sparsetriton/nn/functional/conv/kmap.py:477-484",
        "in_coords": [[0, 1, 1, 1]],
        "spatial_shape": [8, 8, 8],
        "kernel_size": 3, "stride": 1, "padding": 1,
        "out_coords": [[0, 1, 1, 1]],
    },
}

# (name, C_in, C_out, k, stride, padding, dilation, transposed, submanifold, nnz)
CASES = [
    ("subm_k3", 8, 16, 3, 1, 1, 1, False, True, 100),
    ("subm_k5", 8, 16, 5, 1, 2, 1, False, True, 120),
    ("conv_k3s1", 8, 16, 3, 1, 1, 1, False, False, 27),
    ("conv_k3s2", 4, 8, 3, 2, 1, 1, False, False, 27),
    ("conv_k5s2", 16, 16, 5, 2, 2, 1, False, False, 27),
    ("conv_k5s1", 16, 16, 5, 1, 2, 1, False, False, 27),
    ("conv_k3s2d2", 16, 16, 3, 2, 1, 2, False, False, 64),
    ("conv_k3s1p0", 32, 32, 3, 1, 0, 1, False, False, 64),
    ("convT_k3s1", 16, 16, 3, 1, 1, 1, True, False, 27),
    ("convT_k5s1", 8, 8, 5, 1, 2, 1, True, False, 27),
    ("convT_k3s2", 4, 8, 3, 2, 1, 1, True, False, 27),
    ("convT_k3s2b", 8, 16, 3, 2, 1, 1, True, False, 27),
    ("convT_k3s4", 8, 16, 3, 4, 1, 1, True, False, 27),
]


def _dense_case(rng, C_in, C_out, k, s, p, d, transposed, nnz, S=10, B=1):
    lin = np.sort(rng.choice(B * S ** 3, nnz, replace=False))
    coords = np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)
    # Inputs are rounded to float32 so the stored float32 copies are exact.
    feats = rng.standard_normal((nnz, C_in)).astype(np.float32).astype(np.float64)
    weight = (rng.standard_normal((k ** 3, C_in, C_out)) / k ** 1.5).astype(np.float32).astype(np.float64)
    c = torch.as_tensor(coords, dtype=torch.long)
    dense = torch.zeros((B, C_in, S, S, S), dtype=torch.float64)
    dense[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]] = torch.as_tensor(feats)
    dense.requires_grad_(True)
    w = torch.as_tensor(weight).requires_grad_(True)
    if transposed:
        wt = w.view(k, k, k, C_in, C_out).permute(3, 4, 0, 1, 2)
        y = F.conv_transpose3d(dense, wt, stride=s, padding=p, dilation=d)
        occ = F.conv_transpose3d((dense.detach().abs().sum(1, keepdim=True) > 0).double(),
                                 torch.ones((1, 1, k, k, k), dtype=torch.float64), stride=s, padding=p, dilation=d)
    else:
        wt = w.view(k, k, k, C_in, C_out).permute(4, 3, 0, 1, 2)
        y = F.conv3d(dense, wt, stride=s, padding=p, dilation=d)
        occ = F.conv3d((dense.detach().abs().sum(1, keepdim=True) > 0).double(),
                       torch.ones((1, 1, k, k, k), dtype=torch.float64), stride=s, padding=p, dilation=d)
    oc = torch.nonzero(occ[:, 0] > 0)  # (M, 4) sorted lexicographically
    out = y[oc[:, 0], :, oc[:, 1], oc[:, 2], oc[:, 3]]
    dY = torch.as_tensor(rng.standard_normal(tuple(out.shape)).astype(np.float32).astype(np.float64))
    (out * dY).sum().backward()
    dX = dense.grad[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]]
    return dict(coords=coords, feats=feats, weight=weight, out_coords=oc.numpy().astype(np.int32),
                out=out.detach().numpy(), dY=dY.numpy(), dX=dX.numpy(), dW=w.grad.numpy(),
                out_shape=np.array(y.shape[2:], dtype=np.int64), spatial_shape=np.array([S, S, S]))


def main():
    (HERE / "reference_kats.json").write_text(json.dumps(KATS, indent=1))
    rng = np.random.default_rng(20261201)
    arrays = {}
    for name, C_in, C_out, k, s, p, d, tr, subm, nnz in CASES:
        case = _dense_case(rng, C_in, C_out, k, s, p, d, tr, nnz)
        if subm:
            # Keep only the input sites, and redo the gradients for that output set.
            coords = case["coords"]
            S = 10
            c = torch.as_tensor(coords, dtype=torch.long)
            dense = torch.zeros((1, C_in, S, S, S), dtype=torch.float64)
            dense[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]] = torch.as_tensor(case["feats"])
            dense.requires_grad_(True)
            w = torch.as_tensor(case["weight"]).requires_grad_(True)
            y = F.conv3d(dense, w.view(k, k, k, C_in, C_out).permute(4, 3, 0, 1, 2), padding=p, dilation=d)
            out = y[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]]
            dY = torch.as_tensor(rng.standard_normal(tuple(out.shape)).astype(np.float32).astype(np.float64))
            (out * dY).sum().backward()
            case.update(out_coords=coords.copy(), out=out.detach().numpy(), dY=dY.numpy(),
                        dX=dense.grad[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]].numpy(), dW=w.grad.numpy(),
                        out_shape=np.array([S, S, S]))
        meta = np.array([C_in, C_out, k, s, p, d, int(tr), int(subm)], dtype=np.int64)
        arrays[f"{name}/meta"] = meta
        for key, val in case.items():
            if np.asarray(val).dtype == np.float64:
                val = np.asarray(val, dtype=np.float32)  # expected values: float32 storage (rel. 6e-8)
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(HERE / "conv_cases.npz", **arrays)
    print("wrote", HERE / "reference_kats.json", HERE / "conv_cases.npz")


if __name__ == "__main__":
    main()
