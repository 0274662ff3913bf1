"""CPU oracle of the sparse-convolution hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker or the reported CPU
baseline; the product package never does.

Layers:
  * ``liboracle.so`` (``st_oracle.c``, gcc + OpenMP): exact kernel map by
    sort + binary search, first-occurrence output coordinates, float64 GEMMs,
    and a port of the reference's own lossy hash + GEMM algorithm.
  * pure-Python brute force for tiny inputs (dict lookups, explicit loops)
    used to pin the C functions, and dense ``torch.nn.functional.conv3d`` /
    ``conv_transpose3d`` on the CPU in float64 as the independent library
    routine the reference's own tests use (tests/test_sparse_conv.py:37-44).

Every function cites the reference code it restates.  Parity status of each
function (what pins it) is listed in tests/test_oracle.py.
"""

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "st_oracle.c"
LIB = HERE / "_build" / "liboracle.so"

_P = ctypes.c_void_p
_L = ctypes.c_int64
_I = ctypes.c_int
_SIG = {
    "or_exact_kmap": ([_P, _L, _L, _P, _L, _P, _I, _L, _L, _L, _L, _P], _I),
    "or_out_coords": ([_P, _L, _P, _I, _L, _I, _L, _L, _L, _P], _L),
    "or_fwd_f64": ([_P, _I, _P, _I, _I, _P, _L, _P], None),
    "or_dgrad_f64": ([_P, _I, _P, _I, _I, _P, _L, _L, _P], None),
    "or_wgrad_f64": ([_P, _I, _P, _I, _P, _L, _I, _P], None),
    "ref_hash_build": ([_P, _L, _P, _P, _L], _L),
    "ref_hash_query": ([_P, _L, _P, _P, _L, _P], None),
    "ref_kmap": ([_P, _L, _P, _I, _L, _L, _L, _L, _P, _P, _L, _P], None),
    "ref_out_coords": ([_P, _L, _P, _I, _L, _I, _L, _L, _L, _P, _P], _L),
    "ref_fwd_f32": ([_P, _I, _P, _I, _I, _P, _L, _P], None),
    "ref_dgrad_f32": ([_P, _I, _P, _I, _I, _P, _L, _L, _P], None),
    "ref_wgrad_f32": ([_P, _I, _P, _I, _P, _L, _I, _P], None),
    "or_num_threads": ([], _I),
    "or_set_threads": ([_I], None),
}
_lib = None


def build() -> Path:
    """Compile st_oracle.c (gcc, OpenMP) into oracle/_build/liboracle.so."""
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-shared", "-fPIC", str(SRC), "-o", str(tmp)]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        h = ctypes.CDLL(str(LIB))
        for name, (args, res) in _SIG.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = res
        _lib = h
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.int32)


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.float64)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.float32)


# ------------------------------------------------------------ offsets / shapes

def target_offsets(kernel_size: int, dilation: int, padding: int, transposed: bool) -> np.ndarray:
    """(k^3, 3) int32 t_k; input = out*s - t_k (kmap.py:104-180, meshgrid 'ij', x-major)."""
    k, d, p = kernel_size, dilation, padding
    ax = np.arange(k) - k // 2
    gx, gy, gz = np.meshgrid(ax, ax, ax, indexing="ij")
    base = np.stack([gx, gy, gz], axis=-1).reshape(-1, 3) * d
    if transposed:
        t = base - p + (k - 1) * d // 2
    else:
        t = -base + p - (k - 1) * d // 2
    return t.astype(np.int32)


def out_shape(shape, k, s, d, p, transposed):
    """kmap.py:254-258 (normal) and :373-377 (transposed)."""
    if transposed:
        return tuple((v - 1) * s + (k - 1) * d - 2 * p + 1 for v in shape)
    return tuple((v - (k - 1) * d + 2 * p - 1) // s + 1 for v in shape)


# ------------------------------------------------------------- exact (C)

def exact_kmap(in_coords, out_coords, offsets, stride, shape, in_scale=1) -> np.ndarray:
    """(n_out, K) int32 exact neighbour map (conv.py:12-75 with an exact lookup)."""
    ic, oc, off = _i32(in_coords), _i32(out_coords), _i32(offsets)
    n_out, K = oc.shape[0], off.shape[0]
    nbr = np.empty((n_out, K), dtype=np.int32)
    lib().or_exact_kmap(_p(ic), ic.shape[0], in_scale, _p(oc), n_out, _p(off), K, stride, *map(int, shape), _p(nbr))
    return nbr


def out_coords(in_coords, offsets, stride, transposed, new_shape) -> np.ndarray:
    """Output coordinates in first-occurrence order (kmap.py:213-444)."""
    ic, off = _i32(in_coords), _i32(offsets)
    n, K = ic.shape[0], off.shape[0]
    buf = np.empty((max(n * K, 1), 4), dtype=np.int32)
    m = lib().or_out_coords(_p(ic), n, _p(off), K, stride, 1 if transposed else 0, new_shape[0] - 1,
                            new_shape[1] - 1, new_shape[2] - 1, _p(buf))
    return buf[:m].copy()


def fwd_f64(X, W, nbr) -> np.ndarray:
    X, W, nbr = _f64(X), _f64(W), _i32(nbr)
    K, Cin, Cout = W.shape
    out = np.empty((nbr.shape[0], Cout), dtype=np.float64)
    lib().or_fwd_f64(_p(X), Cin, _p(W), K, Cout, _p(nbr), nbr.shape[0], _p(out))
    return out


def dgrad_f64(dY, W, nbr, n_in) -> np.ndarray:
    dY, W, nbr = _f64(dY), _f64(W), _i32(nbr)
    K, Cin, Cout = W.shape
    dX = np.empty((n_in, Cin), dtype=np.float64)
    lib().or_dgrad_f64(_p(dY), Cout, _p(W), K, Cin, _p(nbr), nbr.shape[0], n_in, _p(dX))
    return dX


def wgrad_f64(X, dY, nbr, K) -> np.ndarray:
    X, dY, nbr = _f64(X), _f64(dY), _i32(nbr)
    Cin, Cout = X.shape[1], dY.shape[1]
    dW = np.empty((K, Cin, Cout), dtype=np.float64)
    lib().or_wgrad_f64(_p(X), Cin, _p(dY), Cout, _p(nbr), nbr.shape[0], K, _p(dW))
    return dW


def _valid_pairs(nbr, k):
    o = np.nonzero(nbr[:, k] >= 0)[0]
    return nbr[o, k].astype(np.int64), o


def fwd_f64_blas(X, W, nbr) -> np.ndarray:
    """fwd_f64 as one float64 matrix product per offset (BLAS): the benchmark-size checker.
    out[o] = sum_k X[nbr[o, k]] @ W[k] (implicit_precomputed_gemm.py:64-126)."""
    X, W, nbr = _f64(X), _f64(W), _i32(nbr)
    out = np.zeros((nbr.shape[0], W.shape[2]), dtype=np.float64)
    for k in range(W.shape[0]):
        i, o = _valid_pairs(nbr, k)
        out[o] += X[i] @ W[k]  # o is unique within one offset
    return out


def dgrad_f64_blas(dY, W, nbr, n_in) -> np.ndarray:
    """dgrad_f64 per offset (BLAS): dX[nbr[o, k]] += dY[o] @ W[k]^T, the reference's scatter
    (implicit_precomputed_gemm.py:129-177); rows repeated within one offset accumulate."""
    dY, W, nbr = _f64(dY), _f64(W), _i32(nbr)
    dX = np.zeros((n_in, W.shape[1]), dtype=np.float64)
    for k in range(W.shape[0]):
        i, o = _valid_pairs(nbr, k)
        contrib = dY[o] @ W[k].T
        if np.unique(i).shape[0] == i.shape[0]:
            dX[i] += contrib
        else:
            np.add.at(dX, i, contrib)
    return dX


def wgrad_f64_blas(X, dY, nbr, K) -> np.ndarray:
    """wgrad_f64 per offset (BLAS): dW[k] = sum over pairs X[nbr[o, k]]^T dY[o]
    (implicit_precomputed_gemm.py:180-230)."""
    X, dY, nbr = _f64(X), _f64(dY), _i32(nbr)
    dW = np.zeros((K, X.shape[1], dY.shape[1]), dtype=np.float64)
    for k in range(K):
        i, o = _valid_pairs(nbr, k)
        dW[k] = X[i].T @ dY[o]
    return dW


# ------------------------------------------------- reference-algorithm port

class RefHash:
    """Port of the reference HashTable (utils/hash.py:116-299): 31-bit keys, 128-probe cap, T = int(1.5 N)."""

    def __init__(self, coords, factor: float = 1.5):
        c = _i32(coords)
        self.T = max(int(c.shape[0] * factor), 1)
        self.keys = np.empty(self.T, dtype=np.int32)
        self.vals = np.empty(self.T, dtype=np.int32)
        self.dropped = int(lib().ref_hash_build(_p(c), c.shape[0], _p(self.keys), _p(self.vals), self.T))

    def query(self, coords) -> np.ndarray:
        c = _i32(coords)
        out = np.empty(c.shape[0], dtype=np.int32)
        lib().ref_hash_query(_p(c), c.shape[0], _p(self.keys), _p(self.vals), self.T, _p(out))
        return out

    def kmap(self, out_coords, offsets, stride, shape) -> np.ndarray:
        oc, off = _i32(out_coords), _i32(offsets)
        nbr = np.empty((oc.shape[0], off.shape[0]), dtype=np.int32)
        lib().ref_kmap(_p(oc), oc.shape[0], _p(off), off.shape[0], stride, *map(int, shape), _p(self.keys),
                       _p(self.vals), self.T, _p(nbr))
        return nbr


def ref_out_coords(in_coords, offsets, stride, transposed, new_shape):
    """Output coordinates through the reference's own dedup (kmap.py:213-444, filter_unique_kernel
    :56-97), lossy 31-bit key2 and 1024-probe cap included, candidates resolved one at a time in
    order.  Returns (coords, exhausted) -- exhausted counts candidates that ran out of probes."""
    ic, off = _i32(in_coords), _i32(offsets)
    n, K = ic.shape[0], off.shape[0]
    buf = np.empty((max(n * K, 1), 4), dtype=np.int32)
    ex = ctypes.c_int64()
    m = lib().ref_out_coords(_p(ic), n, _p(off), K, stride, 1 if transposed else 0, *map(int, new_shape), _p(buf),
                             ctypes.byref(ex))
    return buf[:m].copy(), int(ex.value)


def _key_rows(c: np.ndarray) -> np.ndarray:
    c = np.asarray(c, dtype=np.int64)
    return (c[:, 0] << 48) | ((c[:, 1] & 0xFFFF) << 32) | ((c[:, 2] & 0xFFFF) << 16) | (c[:, 3] & 0xFFFF)


def map_ledger(ref_nbr, exact_nbr) -> dict:
    """Entry-by-entry comparison of a kernel map built by the reference's algorithm with the exact
    one over the same output rows: missing (exact has a row, reference -1), false (reference has a
    row where there is none) and wrong (both present, different rows)."""
    r, e = np.asarray(ref_nbr), np.asarray(exact_nbr)
    return {"entries": int((e >= 0).sum()), "missing": int(((e >= 0) & (r < 0)).sum()),
            "false": int(((e < 0) & (r >= 0)).sum()), "wrong": int(((e >= 0) & (r >= 0) & (e != r)).sum())}


def ledger(in_coords, shape, kernel_size=3, stride=1, padding=1, transposed=False, submanifold=True) -> dict:
    """Defect ledger of the reference's lossy hash on one convolution geometry: what its table
    build drops (128-probe cap, utils/hash.py:240-258), what its dedup loses (output coordinates
    whose key2 aliases an earlier one, kmap.py:56-97), and how its kernel map
    (conv.py:12-75 over that table, lossy key2 lookups) differs from the exact map over the
    reference's own output rows.  Inserts and candidates run one at a time in order (the GPU
    runs them in lockstep blocks, so which of two colliding keys wins can differ there)."""
    c = _i32(in_coords)
    off = target_offsets(kernel_size, 1, padding, transposed)
    scale = stride if (transposed and stride > 1) else 1
    table_coords = c.copy()
    table_coords[:, 1:] *= scale
    h = RefHash(table_coords)
    out = {"n_in": int(c.shape[0]), "table_slots": h.T, "insert_dropped": h.dropped}
    lookup_shape = tuple(int(v) * scale for v in shape)
    if submanifold and stride == 1:
        oc = c
        out["n_out"] = int(c.shape[0])
    else:
        ns = out_shape(shape, kernel_size, stride, 1, padding, transposed)
        oc, exhausted = ref_out_coords(c, off, stride, transposed, ns)
        exact_oc = out_coords(c, off, stride, transposed, ns)
        ek, rk = _key_rows(exact_oc), _key_rows(oc)
        out.update({"n_out": int(exact_oc.shape[0]), "ref_n_out": int(oc.shape[0]),
                    "outputs_lost": int(np.setdiff1d(ek, rk).shape[0]),
                    "outputs_spurious": int(np.setdiff1d(rk, ek).shape[0]),
                    "dedup_probe_exhausted": exhausted,
                    "same_order_as_first_occurrence": bool(oc.shape == exact_oc.shape and (oc == exact_oc).all())})
    map_stride = 1 if transposed else stride
    ref_nbr = h.kmap(oc, off, map_stride, lookup_shape)
    if transposed:
        exact = exact_kmap(c, oc, off, 1, lookup_shape, in_scale=scale)
    else:
        exact = exact_kmap(c, oc, off, map_stride, shape)
    out.update(map_ledger(ref_nbr, exact))
    return out


def ref_fwd_f32(X, W, nbr):
    X, W, nbr = _f32(X), _f32(W), _i32(nbr)
    K, Cin, Cout = W.shape
    out = np.empty((nbr.shape[0], Cout), dtype=np.float32)
    lib().ref_fwd_f32(_p(X), Cin, _p(W), K, Cout, _p(nbr), nbr.shape[0], _p(out))
    return out


def ref_dgrad_f32(dY, W, nbr, n_in):
    dY, W, nbr = _f32(dY), _f32(W), _i32(nbr)
    K, Cin, Cout = W.shape
    dX = np.empty((n_in, Cin), dtype=np.float32)
    lib().ref_dgrad_f32(_p(dY), Cout, _p(W), K, Cin, _p(nbr), nbr.shape[0], n_in, _p(dX))
    return dX


def ref_wgrad_f32(X, dY, nbr, K):
    X, dY, nbr = _f32(X), _f32(dY), _i32(nbr)
    Cin, Cout = X.shape[1], dY.shape[1]
    dW = np.empty((K, Cin, Cout), dtype=np.float32)
    lib().ref_wgrad_f32(_p(X), Cin, _p(dY), Cout, _p(nbr), nbr.shape[0], K, _p(dW))
    return dW


def num_threads() -> int:
    return int(lib().or_num_threads())


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


# --------------------------------------------------- brute force (tiny inputs)

def bf_kmap(in_coords, out_coords, offsets, stride, shape, in_scale=1) -> np.ndarray:
    """Dictionary lookup, one (o, k) at a time (conv.py:41-73 semantics)."""
    idx = {}
    for i, (b, x, y, z) in enumerate(np.asarray(in_coords).tolist()):
        idx.setdefault((b, x * in_scale, y * in_scale, z * in_scale), i)
    offs = np.asarray(offsets).tolist()
    res = np.full((len(out_coords), len(offs)), -1, dtype=np.int32)
    for o, (b, x, y, z) in enumerate(np.asarray(out_coords).tolist()):
        for k, (tx, ty, tz) in enumerate(offs):
            q = (x * stride - tx, y * stride - ty, z * stride - tz)
            if all(0 <= q[a] < shape[a] for a in range(3)):
                res[o, k] = idx.get((b,) + q, -1)
    return res


def bf_out_coords(in_coords, offsets, stride, transposed, new_shape, chunk=None) -> np.ndarray:
    """Explicit candidate loop with a seen-set (kmap.py:278-330, 397-444): offset chunks of `chunk`
    offsets in turn (all offsets in one chunk by default), input-major and offset-minor inside a chunk,
    one seen-set across chunks (the reference's global dedup table)."""
    seen, out = set(), []
    offs = np.asarray(offsets).tolist()
    step = len(offs) if not chunk else int(chunk)
    for c0 in range(0, len(offs), step):
        out.extend(_bf_chunk(in_coords, offs[c0:c0 + step], stride, transposed, new_shape, seen))
    return np.asarray(out, dtype=np.int32).reshape(-1, 4)


def _bf_chunk(in_coords, offs, stride, transposed, new_shape, seen):
    out = []
    for b, x, y, z in np.asarray(in_coords).tolist():
        for tx, ty, tz in offs:
            if transposed:
                c = (x * stride + tx, y * stride + ty, z * stride + tz)
            else:
                c = (x + tx, y + ty, z + tz)
                if any(v % stride for v in c):  # Python floor-mod, as torch's `%`
                    continue
                c = tuple(v // stride for v in c)
            if not all(0 <= c[a] <= new_shape[a] - 1 for a in range(3)):
                continue
            key = (b,) + c
            if key not in seen:
                seen.add(key)
                out.append(key)
    return out


def dense_conv_at(in_coords, feats, weight, kernel_size, stride, padding, dilation, transposed, out_coords,
                  spatial_shape):
    """Dense conv3d / conv_transpose3d (float64, CPU) read at out_coords -- tests/test_sparse_conv.py:37-44, 69-76."""
    import torch
    import torch.nn.functional as F

    k = kernel_size
    ic = torch.as_tensor(np.asarray(in_coords), dtype=torch.long)
    f = torch.as_tensor(np.asarray(feats), dtype=torch.float64)
    w = torch.as_tensor(np.asarray(weight), dtype=torch.float64)
    Cin, Cout = w.shape[1], w.shape[2]
    B = int(ic[:, 0].max().item()) + 1 if ic.shape[0] else 1
    dense = torch.zeros((B, Cin) + tuple(int(v) for v in spatial_shape), dtype=torch.float64)
    if ic.shape[0]:
        dense[ic[:, 0], :, ic[:, 1], ic[:, 2], ic[:, 3]] = f
    if transposed:
        wt = w.view(k, k, k, Cin, Cout).permute(3, 4, 0, 1, 2).contiguous()
        y = F.conv_transpose3d(dense, wt, stride=stride, padding=padding, dilation=dilation)
    else:
        wt = w.view(k, k, k, Cin, Cout).permute(4, 3, 0, 1, 2).contiguous()
        y = F.conv3d(dense, wt, stride=stride, padding=padding, dilation=dilation)
    oc = torch.as_tensor(np.asarray(out_coords), dtype=torch.long)
    return y[oc[:, 0], :, oc[:, 1], oc[:, 2], oc[:, 3]].numpy()


# ------------------------------------------------------------ batch norm

def batch_norm_f64(feats, batch_idx, B, weight=None, bias=None, running_mean=None, running_var=None, training=True,
                   eps=1e-5, momentum=0.1, residual=None, relu=False):
    """Per-sample batch norm (nn/functional/norm.py:66-112) followed by the blocks' residual add and
    ReLU (nn/modules/blocks.py:121-124), float64, one loop per sample.

    Training: each sample's rows are normalised by their own mean and biased variance (sum of centred
    squares over the count, the count clamped to 1); the running statistics become
    (1 - momentum) * running + momentum * (mean over the B samples).  Evaluation: the running statistics.
    Returns (out, running_mean', running_var')."""
    x = np.asarray(feats, dtype=np.float64)
    bi = np.asarray(batch_idx, dtype=np.int64)
    C = x.shape[1]
    w = np.ones(C) if weight is None else np.asarray(weight, dtype=np.float64)
    bb = np.zeros(C) if bias is None else np.asarray(bias, dtype=np.float64)
    rm = None if running_mean is None else np.asarray(running_mean, dtype=np.float64)
    rv = None if running_var is None else np.asarray(running_var, dtype=np.float64)
    if training:
        mean = np.zeros((B, C))
        var = np.zeros((B, C))
        for b in range(B):
            rows = x[bi == b]
            cnt = max(rows.shape[0], 1)
            mean[b] = rows.sum(0) / cnt
            var[b] = ((rows - mean[b]) ** 2).sum(0) / cnt
        if rm is not None:
            rm = (1 - momentum) * rm + momentum * mean.mean(0)
        if rv is not None:
            rv = (1 - momentum) * rv + momentum * var.mean(0)
        m_rows, v_rows = mean[bi], var[bi]
    else:
        m_rows, v_rows = rm[None, :], rv[None, :]
    out = (x - m_rows) / np.sqrt(v_rows + eps) * w + bb
    if residual is not None:
        out = out + np.asarray(residual, dtype=np.float64)
    if relu:
        out = np.maximum(out, 0.0)
    return out, rm, rv


def batch_norm_grads_f64(feats, batch_idx, B, weight, bias, running_mean, running_var, training, dout, eps=1e-5,
                         residual=None, relu=False):
    """(dfeats, dweight, dbias, dresidual) of batch_norm_f64 by torch autograd in float64 on the CPU,
    with the normalisation done by the library routine torch.nn.functional.batch_norm applied sample by
    sample (training) or with the running statistics (evaluation), in place of the reference's
    index_add formulation."""
    import torch
    import torch.nn.functional as F

    x = torch.tensor(np.asarray(feats, dtype=np.float64), requires_grad=True)
    bi = torch.as_tensor(np.asarray(batch_idx, dtype=np.int64))
    C = x.shape[1]
    w = torch.tensor(np.ones(C) if weight is None else np.asarray(weight, dtype=np.float64), requires_grad=True)
    b = torch.tensor(np.zeros(C) if bias is None else np.asarray(bias, dtype=np.float64), requires_grad=True)
    res = None
    if residual is not None:
        res = torch.tensor(np.asarray(residual, dtype=np.float64), requires_grad=True)
    if training:
        xh = torch.zeros_like(x)
        for s in range(B):
            rows = (bi == s).nonzero().flatten()
            if rows.numel():
                xh = xh.index_copy(0, rows, F.batch_norm(x[rows], None, None, training=True, eps=eps))
    else:
        rm = torch.as_tensor(np.asarray(running_mean, dtype=np.float64))
        rv = torch.as_tensor(np.asarray(running_var, dtype=np.float64))
        xh = F.batch_norm(x, rm, rv, training=False, eps=eps)
    out = xh * w + b
    if res is not None:
        out = out + res
    if relu:
        out = torch.relu(out)
    out.backward(torch.as_tensor(np.asarray(dout, dtype=np.float64)))
    return (x.grad.numpy(), w.grad.numpy(), b.grad.numpy(), None if res is None else res.grad.numpy())


def conv_f64_torch(x, w, b, nbr):
    """fwd_f64 (+ bias) as a differentiable float64 torch expression: out = sum_k x[nbr[:, k]] @ w[k]
    (+ b), x (n_in, C_in), w (K, C_in, C_out) torch float64; its autograd is the reference's
    input / weight gradient (implicit_precomputed_gemm.py:129-230) by construction."""
    import torch

    nb = torch.as_tensor(np.asarray(nbr, dtype=np.int64))
    out = torch.zeros((nb.shape[0], w.shape[2]), dtype=torch.float64)
    for k in range(w.shape[0]):
        o = (nb[:, k] >= 0).nonzero().flatten()
        if o.numel():
            out = out.index_add(0, o, x[nb[o, k]] @ w[k])
    return out if b is None else out + b


def batch_norm_f64_torch(x, batch_idx, B, w, b, residual=None, relu=False, eps=1e-5):
    """batch_norm_f64 (training statistics) as a differentiable float64 torch expression, by the
    library routine F.batch_norm sample by sample (nn/functional/norm.py:66-112, blocks.py:121-124)."""
    import torch
    import torch.nn.functional as F

    bi = torch.as_tensor(np.asarray(batch_idx, dtype=np.int64))
    xh = torch.zeros_like(x)
    for s in range(B):
        rows = (bi == s).nonzero().flatten()
        if rows.numel():
            xh = xh.index_copy(0, rows, F.batch_norm(x[rows], None, None, training=True, eps=eps))
    out = xh * w + b
    if residual is not None:
        out = out + residual
    return torch.relu(out) if relu else out


# ------------------------------------------------------------ pooling, upsampling

def pool_f64(coords, feats, kernel_size, padding, stride, mode):
    """Sparse pooling (nn/functional/spatial.py:90-135): row r goes to the cell
    floor((coord + padding - kernel_size // 2) / stride); outputs are the distinct cells in ascending
    (b, x, y, z) order, each the max or the mean of its rows.  Cells are kept exact (negative ones too).
    Returns (out_coords, out_feats, inv) with inv[r] = output of row r."""
    c = np.asarray(coords, dtype=np.int64)
    f = np.asarray(feats, dtype=np.float64)
    cells = np.concatenate([c[:, :1], np.floor_divide(c[:, 1:] + padding - kernel_size // 2, stride)], 1)
    uniq, inv = np.unique(cells, axis=0, return_inverse=True)
    inv = inv.reshape(-1)
    out = np.full((uniq.shape[0], f.shape[1]), -np.inf if mode == "max" else 0.0)
    cnt = np.zeros(uniq.shape[0])
    for r in range(c.shape[0]):
        o = inv[r]
        out[o] = np.maximum(out[o], f[r]) if mode == "max" else out[o] + f[r]
        cnt[o] += 1
    if mode == "avg":
        out = out / cnt[:, None]
    return uniq, out, inv


def pool_grad_f64(feats, out, inv, dout, mode):
    """Gradient of pool_f64 as the reference defines it (spatial.py:139-209): each row receives its
    output's gradient, all of it where the row equals the max, or divided by the output's row count."""
    f = np.asarray(feats, dtype=np.float64)
    g = np.asarray(dout, dtype=np.float64)[inv]
    if mode == "max":
        return np.where(f == np.asarray(out, dtype=np.float64)[inv], g, 0.0)
    cnt = np.bincount(inv, minlength=np.asarray(dout).shape[0])
    return g / cnt[inv][:, None]


def upsample_f64(coords, feats, s):
    """Sparse upsampling (spatial.py:236-436): row r becomes rows r s^3 + q, q = (dx s + dy) s + dz, at
    coord * s + (dx, dy, dz)."""
    c = np.asarray(coords, dtype=np.int64)
    f = np.asarray(feats, dtype=np.float64)
    d = np.array([(dx, dy, dz) for dx in range(s) for dy in range(s) for dz in range(s)], dtype=np.int64)
    oc = np.repeat(c, s ** 3, axis=0)
    oc[:, 1:] = oc[:, 1:] * s + np.tile(d, (c.shape[0], 1))
    return oc, np.repeat(f, s ** 3, axis=0)
