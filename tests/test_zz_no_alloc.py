"""hy3x_layer_forward_static: the forward on the library's static per-GPU
scratch, with no allocation. Checked through the C ABI against
hy3x_layer_forward on the same inputs, bit for bit: two calls in a row, the
second with fewer tokens (the array keeps the first call's contents), on both
the decode kernels (T = 1) and the MFMA tiles. Needs an MI355X: marked gpu."""
import ctypes

import numpy as np
import pytest

import hy3_amd as H
from hy3_amd import configs as C

pytestmark = pytest.mark.gpu
STATIC_MAX = 64


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def layer(torch):
    L = H.MoELayer(STATIC_MAX)
    L.synth_experts(C.WEIGHT_SEED, 0)
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    L.set_router(nw, rt, b)
    yield L
    L.close()


def run(torch, L, x, static, K=8):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).copy()).cuda()
    T = x.shape[0]
    fn = H.lib().hy3x_layer_forward_static if static else H.lib().hy3x_layer_forward
    rc = fn(L._h, xd.data_ptr(), T, K, ctypes.c_float(H.ROUTE_SCALE), None)
    assert rc == 0, H.lib().hy3x_last_error().decode()
    torch.cuda.synchronize()
    ids, wpre, w = L.last_routing(T, K)
    return xd.cpu().numpy(), ids, wpre, w


@pytest.mark.parametrize("T1,T2,K", [(48, 5, 8), (64, 1, 8), (1, 1, 4), (33, 17, 2)])
def test_static_equals_forward_twice(torch, layer, T1, T2, K):
    for T, seed in ((T1, 0xD0), (T2, 0xD1)):
        x = C.inputs(seed, T, first_token=T1)
        ref = run(torch, layer, x, static=False, K=K)
        got = run(torch, layer, x, static=True, K=K)
        for a, b in zip(ref, got):
            assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_static_allocates_nothing(torch, layer):
    """After a first call (which looks the array's address up), further calls
    leave the device's free memory unchanged."""
    x = C.inputs(0xD2, 40)
    run(torch, layer, x, static=True)
    xd = torch.from_numpy(x.copy()).cuda()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free0, _ = torch.cuda.mem_get_info()
    for T in (40, 7, 1):
        layer.forward_static(xd.data_ptr(), T)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0


def test_static_rejects_too_many_tokens(torch, layer):
    big = H.MoELayer(STATIC_MAX + 1)
    try:
        x = torch.zeros((STATIC_MAX + 1) * 4096, dtype=torch.float32, device="cuda")
        with pytest.raises(H.HY3XError, match="static"):
            big.forward_static(x.data_ptr(), STATIC_MAX + 1)
        with pytest.raises(H.HY3XError):
            layer.forward_static(x.data_ptr(), 0)
    finally:
        big.close()
