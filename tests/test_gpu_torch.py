"""Torch modules on the fused kernels (run on an MI355X).

Re-runs the reference's tests/test_torch_interop.py on CPU tensors, and checks the
device-tensor path (no NumPy round trip) against the float64 oracle: forward at the
fp32 / fp16 bars (1e-4 / 2e-2), gradients of x and of every parameter at 1e-4,
re-tiling after an in-place optimizer step, padded input rows.
"""
import numpy as np
import pytest

from oracle import kan_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def cuda(gpu):
    if not torch.cuda.is_available():
        pytest.skip("torch sees no GPU")
    return torch.device("cuda:0")


def params_of(m):
    W = m.weight.detach().double().cpu().numpy()
    Wb = m.base_weight.detach().double().cpu().numpy() if m.base_weight is not None else None
    b = m.bias_param.detach().double().cpu().numpy() if m.bias_param is not None else None
    return W, Wb, b


def test_reference_interop_tests_cpu_tensors(gpu):
    """tests/test_torch_interop.py of the reference, on CPU tensors (NumPy layer path)."""
    import metal_kans as mk
    layer = mk.TorchMetalKANLinear(4, 8, basis="cheby", degree=4)
    x = torch.randn(16, 4, requires_grad=True)
    y = layer(x)
    assert y.shape == (16, 8) and not torch.isnan(y).any()
    y.sum().backward()
    assert x.grad is not None and x.grad.shape == (16, 4) and not torch.isnan(x.grad).any()
    net = mk.TorchMetalKAN([4, 8, 2], basis="cheby", degree=3)
    assert net(torch.randn(10, 4)).shape == (10, 2)
    fl = mk.TorchMetalKANLinear(6, 4, basis="fastkan", degree=6)
    assert fl(torch.randn(8, 6)).shape == (8, 4)
    with pytest.raises(ValueError):
        mk.TorchMetalKANLinear(4, 4, basis="relu")


@pytest.mark.parametrize("d_in", [16, 13])
def test_device_cheby_forward_and_gradients(cuda, d_in):
    import metal_kans as mk
    torch.manual_seed(0)
    np.random.seed(0)
    m = mk.TorchMetalKANLinear(d_in, 24, basis="cheby", degree=5).to(cuda)
    with torch.no_grad():
        m.bias_param.normal_(0, 0.1)
    x = (torch.rand(3, 11, d_in, device=cuda) * 2.6 - 1.3).requires_grad_(True)
    y = m(x)
    assert y.is_cuda and y.shape == (3, 11, 24)
    W, Wb, b = params_of(m)
    xs = x.detach().double().cpu().numpy().reshape(33, d_in)
    ref = O.kan_forward("cheby", xs, W, Wb, b, {"K": 5})
    assert O.rel_err(y.detach().cpu().numpy().reshape(33, 24), ref) <= 1e-4
    g = torch.randn_like(y)
    y.backward(g)
    dW, dWb, db, dX = O.cheby_backward(g.double().cpu().numpy().reshape(33, 24), xs, W, Wb, True)
    assert O.rel_err(x.grad.cpu().numpy().reshape(33, d_in), dX) <= 1e-4
    assert O.rel_err(m.weight.grad.cpu().numpy(), dW) <= 1e-4
    assert O.rel_err(m.base_weight.grad.cpu().numpy(), dWb) <= 1e-4
    assert O.rel_err(m.bias_param.grad.cpu().numpy(), db) <= 1e-4


def test_device_training_step_retiles(cuda):
    """Five SGD steps on a 12 -> 20 -> 3 network: the optimizer edits the parameters in place, so
    every forward must re-tile them; the loss trajectory must follow the same steps taken with the
    float64 oracle's forward and backward."""
    import metal_kans as mk
    torch.manual_seed(1)
    np.random.seed(1)
    net = mk.TorchMetalKAN([12, 20, 3], basis="cheby", degree=4).to(cuda)
    Q = [list(params_of(layer)) for layer in net.layers]
    opt = torch.optim.SGD(net.parameters(), lr=0.03)
    x = torch.rand(64, 12, device=cuda) * 2 - 1
    target = torch.randn(64, 3, device=cuda)
    xs, ts = x.double().cpu().numpy(), target.double().cpu().numpy()
    for _ in range(5):
        opt.zero_grad()
        loss = ((net(x) - target) ** 2).mean()
        loss.backward()
        assert all(p.grad is not None for p in net.parameters())
        opt.step()
        # the same step with the oracle
        h = [xs]
        for W, Wb, b in Q:
            h.append(O.kan_forward("cheby", h[-1], W, Wb, b, {"K": 4}))
        ref_loss = np.mean((h[-1] - ts) ** 2)
        assert abs(loss.item() - ref_loss) <= 1e-4 * abs(ref_loss)
        dY = 2 * (h[-1] - ts) / h[-1].size
        for li in (1, 0):
            W, Wb, b = Q[li]
            dW, dWb, db, dY = O.cheby_backward(dY, h[li], W, Wb, True)
            Q[li] = [W - 0.03 * dW, Wb - 0.03 * dWb, b - 0.03 * db]
    for layer, (W, Wb, b) in zip(net.layers, Q):
        got = params_of(layer)
        assert O.rel_err(got[0], W) <= 1e-4 and O.rel_err(got[1], Wb) <= 1e-4 and O.rel_err(got[2], b) <= 1e-4


def test_device_rbf_and_bspline_forward(cuda):
    import metal_kans as mk
    np.random.seed(2)
    for basis, K in (("fastkan", 6), ("bspline", 5)):
        m = mk.TorchMetalKANLinear(10, 7, basis=basis, degree=K).to(cuda)
        x = torch.rand(9, 10, device=cuda) * 2.4 - 1.2
        y = m(x).detach().cpu().numpy()
        W, Wb, b = params_of(m)
        L = m.metal_layer
        if basis == "fastkan":
            p = {"grid": np.asarray(L.grid, np.float64), "inv_den": L.inv_denominator}
            kind = "rbf"
        else:
            p = {"G": L.grid_size, "grid_min": float(L.grid_params[0]), "inv_h": float(L.grid_params[1])}
            kind = "bspline"
        ref = O.kan_forward(kind, x.double().cpu().numpy(), W, Wb, b, p)
        assert O.rel_err(y, ref) <= 1e-4
        xr = x.clone().requires_grad_(True)
        with pytest.raises(NotImplementedError):
            m(xr).sum().backward()


def test_device_half_module(cuda):
    import metal_kans as mk
    np.random.seed(3)
    m = mk.TorchMetalKANLinear(32, 16, basis="cheby", degree=9).to(cuda)
    W, Wb, b = params_of(m)
    x = torch.rand(50, 32, device=cuda) * 2 - 1
    ref = O.kan_forward("cheby", x.double().cpu().numpy(), W, Wb, b, {"K": 9})
    m.half()
    y = m(x.half())
    assert y.dtype == torch.float16
    assert O.rel_err(y.float().detach().cpu().numpy(), ref) <= 2e-2
    y32 = m(x)   # fp32 input to the half module: read unrounded, fp32 output
    assert y32.dtype == torch.float32
    assert O.rel_err(y32.detach().cpu().numpy(), ref) <= 2e-2
