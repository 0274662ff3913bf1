"""Per-sample batch norm (+ residual + ReLU) and the blocks / SparseResNet21D on the GPU.

Batch-norm values and gradients are compared with the float64 oracle
(oracle.batch_norm_f64 / batch_norm_grads_f64) as relative Frobenius errors:
fp32 1e-4 (the statistics are fp32 sums), fp16 1e-2, bf16 2e-2.  Rows are in
random sample order, one sample has no rows, and the channel counts cover the
4-wide vector path (C % 4 == 0), the scalar path and more than one column
block (C > 1024).  The blocks and the backbone are compared with the oracle
composition of the float64 convolution and batch norm.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor
from sparsetriton_amd.nn import (SparseBatchNorm, SparseConvBlock, SparseResBlock, SparseResNet21D, ReLU,
                                 SubMConv3D)
from sparsetriton_amd.nn.functional import sparse_batch_norm, sparse_batch_norm_act

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-4, torch.float16: 1e-2, torch.bfloat16: 2e-2}


def _np(a):
    if isinstance(a, torch.Tensor):
        return a.detach().double().cpu().numpy()
    return np.asarray(a, dtype=np.float64)


def rel(a, b):
    a, b = _np(a), _np(b)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _relu_dout(out_gpu, x_q, bi, B, w, b, rm0, rv0, training, r_q, dout, dtype):
    """dout masked by the GPU's own ReLU decisions, after checking they differ from the oracle's only
    at the kink (|pre-activation| within rounding of 0); the oracle's gradient is then taken without ReLU."""
    z, _, _ = O.batch_norm_f64(x_q, bi, B, w, b, rm0, rv0, training, residual=r_q, relu=False)
    mask = _np(out_gpu) > 0
    differ = mask != (z > 0)
    assert np.all(np.abs(z[differ]) < (1e-4 if dtype == torch.float32 else 5e-2))
    return dout * mask


def _case(rng, n, C, B, empty=2):
    bi = rng.integers(0, B, n)
    if empty is not None and B > 2:
        bi[bi == empty] = 0
    coords = np.zeros((n, 4), np.int32)
    coords[:, 0] = bi
    coords[:, 1:] = rng.integers(0, 50, (n, 3))
    x = rng.standard_normal((n, C)) * 2 + 0.5
    return coords, bi, x


def _sp(device, coords, x, dtype, B, grad=True, shape=(50, 50, 50)):
    f = torch.as_tensor(x, device=device).to(dtype)
    if grad:
        f.requires_grad_(True)
    return SparseTensor(f, torch.as_tensor(coords, device=device), spatial_shape=shape, batch_size=B), f


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("C", [16, 64, 128, 3, 20, 1030])
@pytest.mark.parametrize("residual,relu", [(False, False), (True, True)])
def test_bn_training_vs_oracle(device, dtype, C, residual, relu):
    rng = np.random.default_rng(C * 7 + residual)
    n, B = 3000 if C < 1000 else 700, 4
    coords, bi, x = _case(rng, n, C, B)
    sp, f = _sp(device, coords, x, dtype, B)
    w = torch.as_tensor(rng.standard_normal(C), device=device, dtype=torch.float32).requires_grad_(True)
    b = torch.as_tensor(rng.standard_normal(C), device=device, dtype=torch.float32).requires_grad_(True)
    rm0, rv0 = rng.standard_normal(C), rng.uniform(0.5, 2.0, C)
    rm = torch.as_tensor(rm0, device=device, dtype=torch.float32)
    rv = torch.as_tensor(rv0, device=device, dtype=torch.float32)
    res_np = rng.standard_normal((n, C)) if residual else None
    res = torch.as_tensor(res_np, device=device).to(dtype).requires_grad_(True) if residual else None
    out = sparse_batch_norm_act(sp, w, b, rm, rv, training=True, momentum=0.1, residual=res, relu=relu)
    x_q = f.detach().double().cpu().numpy()  # the inputs as the kernel saw them
    r_q = res.detach().double().cpu().numpy() if residual else None
    ref, ref_rm, ref_rv = O.batch_norm_f64(x_q, bi, B, w.detach().cpu().numpy(), b.detach().cpu().numpy(), rm0, rv0,
                                           True, residual=r_q, relu=relu)
    assert rel(out.F.detach().cpu(), ref) < TOL[dtype]
    assert rel(rm.cpu(), ref_rm) < 1e-5 and rel(rv.cpu(), ref_rv) < 1e-5
    dout = rng.standard_normal((n, C))
    out.F.backward(torch.as_tensor(dout, device=device).to(dtype))
    wn, bn_ = w.detach().cpu().numpy(), b.detach().cpu().numpy()
    dq = _np(torch.as_tensor(dout).to(dtype))
    if relu:
        dq = _relu_dout(out.F, x_q, bi, B, wn, bn_, rm0, rv0, True, r_q, dq, dtype)
    gdx, gdw, gdb, gdres = O.batch_norm_grads_f64(x_q, bi, B, wn, bn_, rm0, rv0, True, dq, residual=r_q)
    tol = 2 * TOL[dtype] if dtype != torch.float32 else 1e-4
    assert rel(f.grad.cpu(), gdx) < tol
    assert rel(w.grad.cpu(), gdw) < tol and rel(b.grad.cpu(), gdb) < tol
    if residual:
        assert rel(res.grad.cpu(), gdres) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("relu", [False, True])
def test_bn_eval_vs_oracle(device, dtype, relu):
    rng = np.random.default_rng(11)
    n, C, B = 2000, 32, 3
    coords, bi, x = _case(rng, n, C, B, empty=None)
    sp, f = _sp(device, coords, x, dtype, B)
    w = torch.as_tensor(rng.standard_normal(C), device=device, dtype=torch.float32).requires_grad_(True)
    b = torch.as_tensor(rng.standard_normal(C), device=device, dtype=torch.float32).requires_grad_(True)
    rm0, rv0 = rng.standard_normal(C), rng.uniform(0.5, 2.0, C)
    rm = torch.as_tensor(rm0, device=device, dtype=torch.float32)
    rv = torch.as_tensor(rv0, device=device, dtype=torch.float32)
    out = sparse_batch_norm_act(sp, w, b, rm, rv, training=False, relu=relu)
    x_q = f.detach().double().cpu().numpy()
    ref, _, _ = O.batch_norm_f64(x_q, bi, B, w.detach().cpu().numpy(), b.detach().cpu().numpy(), rm0, rv0, False,
                                 relu=relu)
    assert rel(out.F.detach().cpu(), ref) < TOL[dtype]
    assert torch.equal(rm.cpu(), torch.as_tensor(rm0, dtype=torch.float32))  # untouched in evaluation
    dout = rng.standard_normal((n, C))
    out.F.backward(torch.as_tensor(dout, device=device).to(dtype))
    wn, bn_ = w.detach().cpu().numpy(), b.detach().cpu().numpy()
    dq = _np(torch.as_tensor(dout).to(dtype))
    if relu:
        dq = _relu_dout(out.F, x_q, bi, B, wn, bn_, rm0, rv0, False, None, dq, dtype)
    gdx, gdw, gdb, _ = O.batch_norm_grads_f64(x_q, bi, B, wn, bn_, rm0, rv0, False, dq)
    tol = 2 * TOL[dtype] if dtype != torch.float32 else 1e-4
    assert rel(f.grad.cpu(), gdx) < tol and rel(w.grad.cpu(), gdw) < tol and rel(b.grad.cpu(), gdb) < tol


def test_bn_many_samples_windows(device):
    # 300 samples x 128 channels exceed one LDS window of sums: the passes run in windows
    rng = np.random.default_rng(12)
    n, C, B = 20000, 128, 300
    coords, bi, x = _case(rng, n, C, B, empty=5)
    sp, f = _sp(device, coords, x, torch.float32, B)
    out = sparse_batch_norm(sp, None, None, None, None, training=True)
    ref, _, _ = O.batch_norm_f64(x, bi, B, training=True)
    assert rel(out.F.detach().cpu(), ref) < 1e-4
    dout = rng.standard_normal((n, C))
    out.F.backward(torch.as_tensor(dout, device=device, dtype=torch.float32))
    gdx, _, _, _ = O.batch_norm_grads_f64(x, bi, B, None, None, None, None, True, dout)
    assert rel(f.grad.cpu(), gdx) < 1e-4


def test_bn_large_offset_moments(device):
    """Features with a mean 1000x their spread: the variance pass sums squares of deviations
    from the sample mean, so it stays accurate where E[y^2] - mean^2 in fp32 would not."""
    rng = np.random.default_rng(14)
    n, C, B = 40000, 32, 3
    coords, bi, x = _case(rng, n, C, B, empty=None)
    x = x * 0.5 + 1000.0 + np.arange(B)[bi][:, None] * 10.0
    sp, _ = _sp(device, coords, x, torch.float32, B, grad=False)
    rm, rv = torch.zeros(C, device=device), torch.ones(C, device=device)
    out = sparse_batch_norm(sp, None, None, rm, rv, training=True, momentum=1.0)
    x_q = sp.F.double().cpu().numpy()
    ref, ref_rm, ref_rv = O.batch_norm_f64(x_q, bi, B, None, None, np.zeros(C), np.ones(C), True, momentum=1.0)
    assert rel(out.F.cpu(), ref) < 1e-4
    assert rel(rm.cpu(), ref_rm) < 1e-6 and rel(rv.cpu(), ref_rv) < 1e-4


def test_bn_deterministic_and_empty(device):
    rng = np.random.default_rng(13)
    coords, bi, x = _case(rng, 50000, 64, 4)
    sp, _ = _sp(device, coords, x, torch.float32, 4, grad=False)
    a = sparse_batch_norm(sp, training=True).F
    b = sparse_batch_norm(sp, training=True).F
    assert torch.equal(a, b)
    # the backward statistics (rows of the 4 samples interleaved at random) are deterministic too
    dout = torch.as_tensor(rng.standard_normal((50000, 64)), device=device, dtype=torch.float32)
    grads = []
    for _ in range(2):
        sp2, f2 = _sp(device, coords, x, torch.float32, 4)
        w2 = torch.ones(64, device=device, requires_grad=True)
        sparse_batch_norm(sp2, w2, None, training=True).F.backward(dout)
        grads.append((f2.grad.clone(), w2.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    rm = torch.zeros(64, device=device)
    rv = torch.ones(64, device=device)
    empty = SparseTensor(torch.zeros((0, 64), device=device), torch.zeros((0, 4), dtype=torch.int32, device=device),
                         spatial_shape=(4, 4, 4), batch_size=2)
    out = sparse_batch_norm(empty, None, None, rm, rv, training=True, momentum=0.5)
    assert out.F.shape == (0, 64)
    # no rows: each sample's mean and variance are 0, so the running statistics decay towards 0
    assert torch.allclose(rm.cpu(), torch.zeros(64)) and torch.allclose(rv.cpu(), torch.full((64,), 0.5))


def test_batch_norm_module_matches_functional(device):
    rng = np.random.default_rng(14)
    coords, bi, x = _case(rng, 4000, 32, 3)
    sp, _ = _sp(device, coords, x, torch.float32, 3, grad=False)
    bn = SparseBatchNorm(32).to(device)
    with torch.no_grad():
        bn.weight.uniform_(0.5, 1.5)
        bn.bias.uniform_(-0.5, 0.5)
    out = bn(sp)
    assert int(bn.num_batches_tracked) == 1
    ref, ref_rm, ref_rv = O.batch_norm_f64(x, bi, 3, bn.weight.detach().cpu().numpy(), bn.bias.detach().cpu().numpy(),
                                           np.zeros(32), np.ones(32), True)
    assert rel(out.F.cpu(), ref) < 1e-4 and rel(bn.running_mean.cpu(), ref_rm) < 1e-5
    bn.eval()
    out_e = bn(sp)
    ref_e, _, _ = O.batch_norm_f64(x, bi, 3, bn.weight.detach().cpu().numpy(), bn.bias.detach().cpu().numpy(),
                                   ref_rm, ref_rv, False)
    assert rel(out_e.F.cpu(), ref_e) < 1e-4


# ------------------------------------------------------------ blocks and backbone

def _rand_set(rng, B=2, S=24, n=1500):
    lin = np.sort(rng.choice(B * S ** 3, n, replace=False))
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32), (S, S, S)


def _conv_oracle(coords, feats, conv, shape):
    """Float64 sparse conv of a module (SubMConv3D with its stride) at the GPU's output order."""
    k, s, d = conv.kernel_size[0], conv.stride[0], conv.dilation[0]
    p = ((k - 1) * d) // 2
    off = O.target_offsets(k, d, p, False)
    if s == 1:
        oc, new_shape = coords, shape
    else:
        new_shape = O.out_shape(shape, k, s, d, p, False)
        oc = O.out_coords(coords, off, s, False, new_shape)
    nbr = O.exact_kmap(coords, oc, off, s, shape)
    W = conv.weight.detach().double().cpu().numpy()
    y = O.fwd_f64(feats, W, nbr)
    if conv.bias is not None:
        y = y + conv.bias.detach().double().cpu().numpy()
    return oc, y, tuple(int(v) for v in new_shape)


def _bn_oracle(bn, bi, B, y, residual=None, relu=False):
    out, _, _ = O.batch_norm_f64(y, bi, B, bn.weight.detach().cpu().numpy(), bn.bias.detach().cpu().numpy(),
                                 np.zeros(y.shape[1]), np.ones(y.shape[1]), True, residual=residual, relu=relu)
    return out


def _block_oracle(block, coords, feats, shape, B):
    if isinstance(block, SparseConvBlock):
        oc, y, ns = _conv_oracle(coords, feats, block[0], shape)
        return oc, _bn_oracle(block[1], oc[:, 0], B, y, relu=True), ns
    m = block.main
    oc, h, ns = _conv_oracle(coords, feats, m[0], shape)
    h = _bn_oracle(m[1], oc[:, 0], B, h, relu=True)
    _, h, _ = _conv_oracle(oc, h, m[3], ns)
    assert isinstance(block.shortcut, torch.nn.Identity)
    return oc, _bn_oracle(m[4], oc[:, 0], B, h, residual=feats, relu=True), ns


def _randomise_bn(model, rng):
    for mod in model.modules():
        if isinstance(mod, SparseBatchNorm):
            with torch.no_grad():
                mod.weight.copy_(torch.as_tensor(rng.uniform(0.5, 1.5, mod.num_features)))
                mod.bias.copy_(torch.as_tensor(rng.uniform(-0.3, 0.3, mod.num_features)))


@pytest.mark.parametrize("kind", ["conv", "res"])
def test_block_fused_matches_oracle_and_unfused(device, kind):
    rng = np.random.default_rng(21 if kind == "conv" else 22)
    torch.manual_seed(0)
    coords, shape = _rand_set(rng)
    C = 16
    x = rng.standard_normal((coords.shape[0], C))
    block = (SparseConvBlock(C, 32, 3, stride=2) if kind == "conv" else SparseResBlock(C, C, 3)).to(device)
    _randomise_bn(block, rng)
    sp, f = _sp(device, coords, x, torch.float32, 2, shape=shape)
    out = block(sp)
    oc, ref, _ = _block_oracle(block, coords, x, shape, 2)
    assert np.array_equal(out.C.cpu().numpy(), oc)
    assert rel(out.F.detach().cpu(), ref) < 2e-3
    # unfused: the same children one after another
    sp2, f2 = _sp(device, coords, x, torch.float32, 2, shape=shape)
    if kind == "conv":
        h = block[2](block[1](block[0](sp2)))
    else:
        h = block.relu(block.main(sp2) + block.shortcut(sp2))
    assert rel(out.F.detach().cpu(), h.F.detach().cpu()) < 1e-5
    dout = torch.as_tensor(rng.standard_normal(tuple(out.F.shape)), device=device, dtype=torch.float32)
    out.F.backward(dout)
    h.F.backward(dout)
    assert rel(f.grad.cpu(), f2.grad.cpu()) < 1e-4


def _f64_params(module):
    """float64 CPU leaf copies of a module's parameters, keyed by the parameter's id."""
    return {id(p): torch.tensor(p.detach().double().cpu().numpy(), requires_grad=True) for p in module.parameters()}


def _conv_torch(conv, P, coords, x_t, shape):
    k, s, d = conv.kernel_size[0], conv.stride[0], conv.dilation[0]
    p = ((k - 1) * d) // 2
    off = O.target_offsets(k, d, p, False)
    if s == 1:
        oc, new_shape = coords, shape
    else:
        new_shape = O.out_shape(shape, k, s, d, p, False)
        oc = O.out_coords(coords, off, s, False, new_shape)
    nbr = O.exact_kmap(coords, oc, off, s, shape)
    b = None if conv.bias is None else P[id(conv.bias)]
    return oc, O.conv_f64_torch(x_t, P[id(conv.weight)], b, nbr), tuple(int(v) for v in new_shape)


def _block_torch(block, P, coords, x_t, shape, B):
    """The block as a float64 autograd expression of the oracle's convolution and batch norm."""
    if isinstance(block, SparseConvBlock):
        oc, y, ns = _conv_torch(block[0], P, coords, x_t, shape)
        bn = block[1]
        return oc, O.batch_norm_f64_torch(y, oc[:, 0], B, P[id(bn.weight)], P[id(bn.bias)], relu=True), ns
    m = block.main
    oc, h, ns = _conv_torch(m[0], P, coords, x_t, shape)
    h = O.batch_norm_f64_torch(h, oc[:, 0], B, P[id(m[1].weight)], P[id(m[1].bias)], relu=True)
    _, h, _ = _conv_torch(m[3], P, oc, h, ns)
    return oc, O.batch_norm_f64_torch(h, oc[:, 0], B, P[id(m[4].weight)], P[id(m[4].bias)], residual=x_t,
                                      relu=True), ns


@pytest.mark.parametrize("kind", ["conv", "res"])
def test_block_backward_vs_f64_autograd(device, kind):
    """Training block (fused batch norm / residual / ReLU kernels): input and every parameter's
    gradient against autograd of the float64 oracle composition.  The tolerance (5e-3) leaves room
    for a ReLU decision that rounding flips at the kink."""
    rng = np.random.default_rng(41 if kind == "conv" else 42)
    torch.manual_seed(0)
    coords, shape = _rand_set(rng)
    C = 16
    x = rng.standard_normal((coords.shape[0], C))
    block = (SparseConvBlock(C, 32, 3, stride=2) if kind == "conv" else SparseResBlock(C, C, 3)).to(device)
    _randomise_bn(block, rng)
    sp, f = _sp(device, coords, x, torch.float32, 2, shape=shape)
    out = block(sp)
    dout = rng.standard_normal(tuple(out.F.shape))
    out.F.backward(torch.as_tensor(dout, device=device, dtype=torch.float32))
    P = _f64_params(block)
    x_t = torch.tensor(x, requires_grad=True)
    oc, ref, _ = _block_torch(block, P, coords, x_t, shape, 2)
    assert np.array_equal(out.C.cpu().numpy(), oc)
    ref.backward(torch.as_tensor(dout))
    assert rel(f.grad, x_t.grad) < 5e-3
    _check_param_grads(block, P, 5e-3)


def _check_param_grads(module, P, tol):
    """Each parameter's gradient within tol of the float64 one, relative to its own norm -- or, for
    a gradient that is zero in exact arithmetic (a convolution bias feeding a training-mode batch
    norm, which removes it), to the largest parameter gradient of the module."""
    ref = {name: _np(P[id(prm)].grad) for name, prm in module.named_parameters()}
    scale = max(np.linalg.norm(g) for g in ref.values())
    errs = {}
    for name, prm in module.named_parameters():
        denom = max(np.linalg.norm(ref[name]), 1e-3 * scale)
        errs[name] = float(np.linalg.norm(_np(prm.grad) - ref[name]) / denom)
    worst = max(errs.items(), key=lambda kv: kv[1])
    assert worst[1] < tol, worst
    return errs


@pytest.mark.parametrize("precision,stages,tol", [("ieee", 5, 1e-4), ("bf16x3", 2, 1e-3)])
def test_resnet21d_backward_vs_f64_autograd(device, precision, stages, tol):
    """SparseResNet21D training step (fp32): input and all 84 parameter gradients (21 convolutions,
    21 batch norms) against autograd of the float64 oracle composition, stage by stage, with a loss
    over the first `stages` stages' outputs.

    The last stages of this small set hold 128 and 16 voxels, and batch norm over so few rows makes
    the gradient ill-conditioned: a relative perturbation of 4.4e-6 on every convolution output of
    the float64 composition itself moves the input gradient by 1.3 % (ReLU decisions flip).  IEEE
    fp32 convolutions (~1e-7) stay clear of that and are checked through all five stages; the
    split-bf16 mode (~4e-6 per convolution, pinned per layer elsewhere) through the first two."""
    from sparsetriton_amd.config import set_fp32_precision

    set_fp32_precision(precision)
    rng = np.random.default_rng(33)
    torch.manual_seed(2)
    coords, shape = _rand_set(rng, B=2, S=32, n=3000)
    x = rng.standard_normal((coords.shape[0], 4))
    model = SparseResNet21D(in_channels=4).to(device)
    _randomise_bn(model, rng)
    sp, f = _sp(device, coords, x, torch.float32, 2, shape=shape)
    outs = model(sp)
    sum(o.F.square().mean() for o in outs[:stages]).backward()
    P = _f64_params(model)
    x_t = torch.tensor(x, requires_grad=True)
    c, h, s = coords, x_t, shape
    ref_outs = []
    for stage in model:
        for block in stage:
            c, h, s = _block_torch(block, P, c, h, s, 2)
        ref_outs.append(h)
    sum(o.square().mean() for o in ref_outs[:stages]).backward()
    for got, want in zip(outs, ref_outs):
        assert rel(got.F.detach(), want.detach()) < tol
    assert rel(f.grad, x_t.grad) < tol
    for prm in model.parameters():  # parameters past the loss's last stage get no gradient
        if P[id(prm)].grad is None:
            assert prm.grad is None or not prm.grad.any()
            P[id(prm)].grad = torch.zeros_like(P[id(prm)])
            prm.grad = torch.zeros_like(prm)
    assert len(_check_param_grads(model, P, tol)) == 84


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_resnet21d_forward_backward(device, dtype):
    rng = np.random.default_rng(31)
    torch.manual_seed(1)
    coords, shape = _rand_set(rng, B=2, S=32, n=3000)
    x = rng.standard_normal((coords.shape[0], 4))
    model = SparseResNet21D(in_channels=4).to(device)
    _randomise_bn(model, rng)
    if dtype != torch.float32:
        for mod in model.modules():
            if isinstance(mod, SubMConv3D):
                mod.to(dtype)
    sp, f = _sp(device, coords, x, dtype, 2, shape=shape)
    outs = model(sp)
    assert len(outs) == 5
    # float64 oracle, stage by stage, block by block (the GPU's output order is the oracle's)
    c, h, s = coords, x, shape
    for stage, got in zip(model, outs):
        for block in stage:
            c, h, s = _block_oracle(block, c, h, s, 2)
        assert np.array_equal(got.C.cpu().numpy(), c)
        assert rel(got.F.detach().float().cpu(), h) < (5e-3 if dtype == torch.float32 else 6e-2)
    loss = sum(o.F.float().square().mean() for o in outs)
    loss.backward()
    assert f.grad is not None and torch.isfinite(f.grad).all()
    for p in model.parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all()


# ------------------------------------------------------- evaluation: fused store epilogue

def _randomise_running(model, rng):
    for mod in model.modules():
        if isinstance(mod, SparseBatchNorm):
            mod.running_mean.copy_(torch.as_tensor(rng.uniform(-0.5, 0.5, mod.num_features)))
            mod.running_var.copy_(torch.as_tensor(rng.uniform(0.5, 2.0, mod.num_features)))


def _bn_eval_oracle(bn, y, residual=None, relu=False):
    out, _, _ = O.batch_norm_f64(y, np.zeros(y.shape[0], np.int64), 1, bn.weight.detach().cpu().numpy(),
                                 bn.bias.detach().cpu().numpy(), bn.running_mean.cpu().numpy(),
                                 bn.running_var.cpu().numpy(), False, residual=residual, relu=relu)
    return out


def _block_eval_oracle(block, coords, feats, shape):
    if isinstance(block, SparseConvBlock):
        oc, y, ns = _conv_oracle(coords, feats, block[0], shape)
        return oc, _bn_eval_oracle(block[1], y, relu=True), ns
    m = block.main
    oc, h, ns = _conv_oracle(coords, feats, m[0], shape)
    h = _bn_eval_oracle(m[1], h, relu=True)
    _, h, _ = _conv_oracle(oc, h, m[3], ns)
    return oc, _bn_eval_oracle(m[4], h, residual=feats, relu=True), ns


@pytest.mark.parametrize("kind", ["conv", "res"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_eval_store_epilogue(device, kind, dtype):
    rng = np.random.default_rng(41 if kind == "conv" else 42)
    torch.manual_seed(2)
    coords, shape = _rand_set(rng)
    C = 32
    x = rng.standard_normal((coords.shape[0], C))
    block = (SparseConvBlock(C, 64, 3, stride=2) if kind == "conv" else SparseResBlock(C, C, 3)).to(device)
    _randomise_bn(block, rng)
    _randomise_running(block, rng)
    for mod in block.modules():
        if isinstance(mod, SubMConv3D):
            mod.to(dtype)
    block.eval()
    sp, _ = _sp(device, coords, x, dtype, 2, grad=False, shape=shape)
    with torch.no_grad():
        out = block(sp)  # fused: one GEMM pass per convolution
        if kind == "conv":
            ref_gpu = block[2](block[1](block[0](sp)))
        else:
            ref_gpu = block.relu(block.main(sp) + block.shortcut(sp))
    oc, ref, _ = _block_eval_oracle(block, coords, _np(sp.F), shape)
    assert np.array_equal(out.C.cpu().numpy(), oc)
    tol = 2e-3 if dtype == torch.float32 else 2e-2
    assert rel(out.F, ref) < tol
    assert rel(out.F, ref_gpu.F) < tol


def test_resnet21d_eval_fused_vs_oracle(device):
    rng = np.random.default_rng(43)
    torch.manual_seed(3)
    coords, shape = _rand_set(rng, B=2, S=32, n=3000)
    x = rng.standard_normal((coords.shape[0], 4))
    model = SparseResNet21D(in_channels=4).to(device)
    _randomise_bn(model, rng)
    _randomise_running(model, rng)
    model.eval()
    sp, _ = _sp(device, coords, x, torch.float32, 2, grad=False, shape=shape)
    with torch.no_grad():
        outs = model(sp)
    c, h, s = coords, x, shape
    for stage, got in zip(model, outs):
        for block in stage:
            c, h, s = _block_eval_oracle(block, c, h, s)
        assert np.array_equal(got.C.cpu().numpy(), c)
        assert rel(got.F, h) < 5e-3


def test_conv_transpose_block_vs_oracle(device):
    """SparseConvTransposeBlock (blocks.py:50-81): transposed conv + batch norm + ReLU, training."""
    from sparsetriton_amd.nn import SparseConvTransposeBlock

    rng = np.random.default_rng(51)
    torch.manual_seed(4)
    coords, shape = _rand_set(rng, B=2, S=12, n=400)
    C = 16
    x = rng.standard_normal((coords.shape[0], C))
    block = SparseConvTransposeBlock(C, 8, 3, stride=2).to(device)
    _randomise_bn(block, rng)
    sp, f = _sp(device, coords, x, torch.float32, 2, shape=shape)
    out = block(sp)
    conv = block[0]
    k, s, p, d = conv.kernel_size[0], conv.stride[0], conv.padding[0], conv.dilation[0]
    off = O.target_offsets(k, d, p, True)
    ns = O.out_shape(shape, k, s, d, p, True)
    oc = out.C.cpu().numpy()
    assert sorted(map(tuple, oc.tolist())) == sorted(map(tuple, O.out_coords(coords, off, s, True, ns).tolist()))
    nbr = O.exact_kmap(coords, oc, off, 1, tuple(v * s for v in shape), in_scale=s)
    y = O.fwd_f64(x, conv.weight.detach().double().cpu().numpy(), nbr) + conv.bias.detach().double().cpu().numpy()
    ref = _bn_oracle(block[1], oc[:, 0], 2, y, relu=True)
    assert rel(out.F, ref) < 2e-3
    # gradient through the fused path equals the unfused children's
    sp2, f2 = _sp(device, coords, x, torch.float32, 2, shape=shape)
    h = block[2](block[1](block[0](sp2)))
    dout = torch.randn(tuple(out.F.shape), device=device)
    out.F.backward(dout)
    h.F.backward(dout)
    assert rel(f.grad, f2.grad) < 1e-4
