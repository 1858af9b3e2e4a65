"""HIP path (libhy3x.so through its C ABI) against the CPU oracle and the
reference fixtures. Needs an MI355X: marked gpu.

Bars: routing bit-exact against the oracle (ids identical, pre-scale weights
bit-identical); against hy3.c's fixtures ids identical and pre-scale weights
within 4 ulp (the reference's RMSNorm scale comes from the host CPU's rsqrt
estimate), and within 1 ulp when the HIP router is given hy3.c's own scale;
MoE output relative L2 <= 1e-3 on the delta y - x and on y.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import hy3_amd as H
from hy3_amd import configs as C
from hy3_amd import hipmem
from oracle import hy3_oracle as O

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D, E = 4096, 192
TOL = 1e-3


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ulp_dist(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def layer(torch):
    L = H.MoELayer(4096)
    L.synth_experts(C.WEIGHT_SEED, 0)
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    L.set_router(nw, rt, b)
    yield L
    L.close()


class DeviceBackedLayer(O.SynthLayer):
    """Oracle layer whose expert bytes are copied from the device arena."""

    def __init__(self, dev_layer, seed, layer=0):
        super().__init__(seed, layer)
        self.dev = dev_layer

    def expert(self, e):
        if e not in self.experts:
            self.experts[e] = tuple(hipmem.to_host(self.dev.expert_ptr(e, m), H.Q4K_MATRIX_BYTES)
                                    for m in range(3))
        return self.experts[e]


@pytest.fixture(scope="module")
def cpu(layer):
    return DeviceBackedLayer(layer, C.WEIGHT_SEED)


def set_bias(layer, cpu, kind, seed=None):
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    if kind == "zipf":
        b = H.synth_zipf_bias(E, seed)
    layer.set_router(nw, rt, None if kind == "none" else b)
    cpu.bias = b.copy()
    cpu.has_bias = kind != "none"


def run(torch, layer, x, K=8):
    T = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).copy()).cuda()
    layer.forward(xd.data_ptr(), T, K)
    torch.cuda.synchronize()
    ids, wpre, w = layer.last_routing(T, K)
    return xd.cpu().numpy(), ids, wpre, w


# ---------------------------------------------------------------- inputs
def test_synth_layer_matches_reference_quantiser(layer):
    """The device generator + quantiser reproduce, for all 579 matrices of the
    layer, the bytes hy3_convert.c's compiled quantize_row_q4_K wrote."""
    with open(os.path.join(G, "layer.json")) as f:
        meta = json.load(f)
    bad = []
    for e in range(E + 1):
        got = [sha(hipmem.to_host(layer.expert_ptr(e, m), H.Q4K_MATRIX_BYTES)) for m in range(3)]
        if got != meta["expert_sha256"][str(e)]:
            bad.append(e)
    assert not bad, f"experts differing from the reference quantiser: {bad}"


def test_small_tensors_match_oracle():
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    ref = O.SynthLayer(C.WEIGHT_SEED)
    assert np.array_equal(nw, ref.norm_w) and np.array_equal(rt.ravel(), ref.router)
    assert np.array_equal(b, ref.bias)
    assert np.array_equal(H.synth_zipf_bias(E, 0xC3), O.zipf_bias(E, 0xC3))
    assert np.array_equal(C.inputs(0xC1, 3, first_token=5).ravel(),
                          O.normal(3 * D, O.key(0xC1, 0, O.T_X), 1.0, first=5 * D))


def test_device_quantiser_edge_blocks(torch):
    f = np.load(os.path.join(G, "q4k_quant.npz"))
    x = torch.from_numpy(f["x"]).cuda()
    q = torch.zeros(f["q"].size, dtype=torch.uint8, device="cuda")
    rc = H.lib().hy3x_synth_quantize_q4k(x.data_ptr(), q.data_ptr(), x.numel(), None)
    assert rc == 0
    torch.cuda.synchronize()
    got = q.cpu().numpy().reshape(-1, 144)
    bad = np.nonzero((got != f["q"].reshape(-1, 144)).any(1))[0]
    assert bad.size == 0, f"blocks differing: {bad.tolist()}"


# ---------------------------------------------------------------- routing
@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_routing_bit_exact_vs_oracle(torch, layer, cpu, cfg):
    c = C.CONFIGS[cfg]
    set_bias(layer, cpu, "zipf" if c.zipf_bias else "uniform", c.input_seed)
    x = C.inputs(c.input_seed, c.T)
    _, ids, wpre, w = run(torch, layer, x)
    r = cpu.route(x)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))
    assert np.array_equal(w.view(np.uint32), r["w"].view(np.uint32))
    set_bias(layer, cpu, "uniform")


@pytest.mark.parametrize("K", [1, 2, 4, 8])
@pytest.mark.parametrize("T", [1, 5, 16])
def test_routing_top_k_variants(torch, layer, cpu, K, T):
    x = C.inputs(0xC2, T, first_token=100)
    _, ids, wpre, _ = run(torch, layer, x, K)
    r = cpu.route(x, K)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))


@pytest.mark.parametrize("T,K", [(64, 8), (65, 8), (256, 8), (257, 3), (512, 8), (513, 5),
                                 (1536, 8), (1537, 6), (2560, 8), (2561, 4)])
def test_routing_at_router_tile_boundaries(torch, layer, cpu, T, K):
    """Every token's routing at both sides of each change of router GEMM tile
    (64 / 256 / 1536 / 2560 tokens) and of the top-K launch shape (256 tokens),
    with the tile edges falling mid-tile (65, 257, 513, 1537, 2561)."""
    x = C.inputs(0xC3, T, first_token=1000)
    _, ids, wpre, w = run(torch, layer, x, K)
    r = cpu.route(x, K)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))
    assert np.array_equal(w.view(np.uint32), r["w"].view(np.uint32))


@pytest.mark.parametrize("T", [319, 320, 1151, 1152])
def test_default_path_thresholds(torch, layer, cpu, T):
    """At both sides of the default path's changes of tile shape (narrow to
    wide tiles at 320 tokens, wide to 128-token tiles at 1152): the layer
    reports the shape it ran, routing is bit-exact and sampled outputs match
    the oracle."""
    x = C.inputs(0xC9, T, first_token=2000)
    y, ids, wpre, _ = run(torch, layer, x)
    assert layer.last_path() == (5 if T >= 1152 else 4 if T >= 320 else 3)
    r = cpu.route(x)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))
    rows = np.linspace(0, T - 1, 4).astype(int)
    yo, _ = cpu.forward(x[rows])
    assert O.rel_l2(y[rows] - x[rows], yo - x[rows]) <= TOL


def test_routing_without_bias(torch, layer, cpu):
    set_bias(layer, cpu, "none")
    x = C.inputs(0xC1, 12)
    _, ids, wpre, _ = run(torch, layer, x)
    r = cpu.route(x)
    set_bias(layer, cpu, "uniform")
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))


# ---------------------------------------------------------------- outputs
@pytest.mark.parametrize("cfg,sample", [(0, None), (1, None), (2, 8), (3, 8)])
def test_output_vs_oracle(torch, layer, cpu, cfg, sample):
    c = C.CONFIGS[cfg]
    set_bias(layer, cpu, "zipf" if c.zipf_bias else "uniform", c.input_seed)
    x = C.inputs(c.input_seed, c.T)
    y, ids, _, _ = run(torch, layer, x)
    rows = np.arange(c.T) if sample is None else np.linspace(0, c.T - 1, sample).astype(int)
    yo, ro = cpu.forward(x[rows])
    set_bias(layer, cpu, "uniform")
    assert np.array_equal(ro["ids"], ids[rows])
    assert O.rel_l2(y[rows] - x[rows], yo - x[rows]) <= TOL
    assert O.rel_l2(y[rows], yo) <= TOL


MOE_CASES = ["c0", "c0_k4", "c0_nobias", "c1", "c2", "c3"]


def reference_wpre(f, name, ids_ref):
    """hy3.c's pre-scale gate weights from its recorded sigmoids, summed in k
    order as hy3.c:1283-1288 does."""
    T, K = ids_ref.shape
    sig = f[f"{name}/sigmoid"][:T]
    sel = sig[np.arange(T)[:, None], ids_ref]
    s = np.zeros(T, np.float32)
    for k in range(K):
        s = (s + sel[:, k]).astype(np.float32)
    return (sel * (np.float32(1) / (s + np.float32(1e-20)))[:, None]).astype(np.float32)


@pytest.mark.parametrize("name", MOE_CASES)
def test_vs_reference_fixtures(torch, layer, cpu, name):
    """Against hy3.c's recorded routing with the contract's own RMSNorm scale:
    ids identical, pre-scale weights within 4 ulp (the largest distance seen
    on these fixtures; all of it comes from hy3.c's r, an rsqrt estimate plus
    a Newton step), outputs within TOL."""
    f = np.load(os.path.join(G, "moe.npz"))
    bk = str(f[f"{name}/bias_kind"][0])
    seed = int(f[f"{name}/x_seed"][0])
    ids_ref = f[f"{name}/ids"]
    T, K = ids_ref.shape
    set_bias(layer, cpu, bk, seed)
    x = C.inputs(seed, T)
    y, ids, wpre, _ = run(torch, layer, x, K)
    set_bias(layer, cpu, "uniform")
    assert np.array_equal(ids, ids_ref)
    assert ulp_dist(wpre, reference_wpre(f, name, ids_ref)).max() <= 4
    y_ref = f[f"{name}/y"]
    n = y_ref.shape[0]
    assert O.rel_l2(y[:n] - x[:n], y_ref - x[:n]) <= TOL
    assert O.rel_l2(y[:n], y_ref) <= TOL


# fixture cases and token counts: T = 1 runs the decode router, 2..8 the
# per-(expert, token) router blocks, > 8 the RMSNorm kernel + router GEMM
RMS_CASES = [("c0", None), ("c0_k4", None), ("c0_nobias", None), ("c1", 5), ("c1", None),
             ("c2", None), ("c3", None)]


@pytest.mark.parametrize("name,T", RMS_CASES)
def test_reference_rms_scale_gives_one_ulp(torch, layer, cpu, name, T):
    """Given hy3.c's own RMSNorm scale r per token (recorded in the fixture,
    hy3.c:435-444 as built), the HIP router reproduces the reference build's
    routing on every fixture token: expert ids identical and pre-scale gate
    weights within 1 ulp (hy3.c:1283-1291), on each router kernel."""
    f = np.load(os.path.join(G, "moe.npz"))
    bk = str(f[f"{name}/bias_kind"][0])
    seed = int(f[f"{name}/x_seed"][0])
    ids_ref = f[f"{name}/ids"][:T]
    T, K = ids_ref.shape
    set_bias(layer, cpu, bk, seed)
    layer.set_rms_scale(f[f"{name}/rms_r"][:T])
    try:
        _, ids, wpre, _ = run(torch, layer, C.inputs(seed, T), K)
    finally:
        layer.set_rms_scale(None)
        set_bias(layer, cpu, "uniform")
    assert np.array_equal(ids, ids_ref)
    assert ulp_dist(wpre, reference_wpre(f, name, ids_ref)).max() <= 1


def test_rms_scale_override_is_switched_off(torch, layer, cpu):
    """After the override is cleared the computed scale is used again: routing
    equals the oracle's bit for bit."""
    x = C.inputs(0xC0, 1)
    layer.set_rms_scale(np.array([0.5], np.float32))
    layer.set_rms_scale(None)
    _, ids, wpre, _ = run(torch, layer, x)
    r = cpu.route(x)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))


def test_last_routing_refused_after_another_layers_forward(torch):
    """Layers sharing one scratch: once layer B has run, layer A's routing is
    gone from the scratch and hy3x_layer_last_routing(A) says so instead of
    returning B's ids."""
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    A = H.MoELayer(4)
    Bl = H.MoELayer(4, share_scratch_with=A)
    try:
        for L in (A, Bl):
            L.synth_experts(C.WEIGHT_SEED, 0)
            L.set_router(nw, rt, b)
        x = torch.from_numpy(C.inputs(0xC0, 2).copy()).cuda()
        A.forward(x.data_ptr(), 2)
        torch.cuda.synchronize()
        A.last_routing(2, 8)
        Bl.forward(x.data_ptr(), 2)
        torch.cuda.synchronize()
        Bl.last_routing(2, 8)
        with pytest.raises(H.HY3XError, match="another layer"):
            A.last_routing(2, 8)
    finally:
        Bl.close()
        A.close()


@pytest.mark.parametrize("T", [1, 5, 40])
def test_rms_scale_override_serves_one_forward(torch, layer, cpu, T):
    """An override left set is consumed by the next forward: the forward after
    it, with no clearing call, routes with the computed scale again (equal to
    the oracle bit for bit), while the overridden forward itself did not."""
    x = C.inputs(0xC1, T)
    r = cpu.route(x)
    layer.set_rms_scale(np.full(T, 0.37, np.float32))
    _, ids0, wpre0, _ = run(torch, layer, x)
    assert not np.array_equal(wpre0.view(np.uint32), r["wpre"].view(np.uint32))
    _, ids, wpre, _ = run(torch, layer, x)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))


@pytest.mark.parametrize("K", [1, 2, 4])
@pytest.mark.parametrize("T,path", [(1, 0), (40, 3), (40, 4), (40, 1), (40, 5), (300, 5)])
def test_output_top_k_variants(torch, layer, cpu, K, T, path):
    """Top-K below 8 through every expert path (decode kernels, narrow, wide
    and 128-token MFMA tiles, GEMV tiles): routing bit-exact, output within
    TOL."""
    x = C.inputs(0xC6, T, first_token=7)
    rows = np.linspace(0, T - 1, min(T, 4)).astype(int)
    layer.set_path(path)
    try:
        y, ids, wpre, _ = run(torch, layer, x, K)
    finally:
        layer.set_path(0)
    yo, ro = cpu.forward(x[rows], K=K)
    assert np.array_equal(ids[rows], ro["ids"])
    assert np.array_equal(wpre[rows].view(np.uint32), ro["wpre"].view(np.uint32))
    assert O.rel_l2(y[rows] - x[rows], yo - x[rows]) <= TOL


def test_forward_argument_errors(torch, layer):
    """Out-of-range T and K are errors with a message; the layer stays usable."""
    x = torch.zeros(4096, dtype=torch.float32, device="cuda")
    for T, K in [(0, 8), (4097, 8), (1, 0), (1, 9)]:
        with pytest.raises(H.HY3XError):
            layer.forward(x.data_ptr(), T, K)
    y, *_ = run(torch, layer, C.inputs(0xC2, 1))
    assert np.isfinite(y).all()


@pytest.mark.parametrize("T", [64, 512])
def test_deterministic_both_shapes(torch, layer, T):
    """Repeated forwards give the same bits on the narrow (T = 64) and the
    wide (T = 512) MFMA tiles."""
    x = C.inputs(0xC7, T)
    y1, *_ = run(torch, layer, x)
    y2, *_ = run(torch, layer, x)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_token_permutation_full_size(torch, layer, cpu):
    """Full-size property at config 3's shape (4096 tokens, Zipf routing):
    permuting the tokens permutes the routing and the outputs exactly. A
    token's arithmetic does not depend on its row in an MFMA tile, on the
    tile's token count or on the other tokens of the batch."""
    c = C.CONFIGS[3]
    set_bias(layer, cpu, "zipf", c.input_seed)
    try:
        x = C.inputs(c.input_seed, c.T)
        perm = np.random.default_rng(5).permutation(c.T)
        y, ids, wpre, _ = run(torch, layer, x)
        yp, idsp, wprep, _ = run(torch, layer, x[perm])
    finally:
        set_bias(layer, cpu, "uniform")
    assert np.array_equal(idsp, ids[perm])
    assert np.array_equal(wprep.view(np.uint32), wpre[perm].view(np.uint32))
    assert np.array_equal(yp.view(np.uint32), y[perm].view(np.uint32))


def test_batch_invariance(torch, layer):
    """For T >= 2 a token's output does not depend on the other tokens of
    its forward: three tokens alone, inside a batch of 40 (narrow tiles) and
    inside a batch of 500 (wide tiles) give the same bits."""
    x = C.inputs(0xC8, 500)
    pick = np.array([3, 17, 33])
    alone, *_ = run(torch, layer, x[pick])
    mid, *_ = run(torch, layer, x[:40])
    big, *_ = run(torch, layer, x)
    assert np.array_equal(alone.view(np.uint32), mid[pick].view(np.uint32))
    assert np.array_equal(alone.view(np.uint32), big[pick].view(np.uint32))


def test_deterministic(torch, layer):
    x = C.inputs(0xC2, 64)
    y1, *_ = run(torch, layer, x)
    y2, *_ = run(torch, layer, x)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_zero_experts_leave_residual_unchanged(torch):
    """Full-size property: all-zero Q4_K blocks dequantise to 0 (scales and
    mins are 0; d decodes to 2^-15 by the fp16 quirk), so y == x exactly."""
    L = H.MoELayer(512)
    z = np.zeros(H.Q4K_MATRIX_BYTES, np.uint8)
    for e in range(E + 1):
        L.set_expert_q4k(e, z, z, z)
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    L.set_router(nw, rt, b)
    x = C.inputs(0xC2, 512)
    y, *_ = run(torch, L, x)
    L.close()
    assert np.array_equal(y.view(np.uint32), x.view(np.uint32))


@pytest.mark.parametrize("T", [1, 16])
@pytest.mark.parametrize("case", ["all_equal", "bias_ties", "some_ties"])
def test_routing_with_ties(torch, T, case):
    """Tied scores: the selection-with-swaps order (hy3.c:654-666) decides, on
    both router paths (decode T=1 and the large-T path)."""
    L = H.MoELayer(16)
    L.synth_experts(C.WEIGHT_SEED, 0)
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    if case == "all_equal":
        rt = np.zeros_like(rt)
        b = np.zeros_like(b)
    elif case == "bias_ties":
        rt = np.zeros_like(rt)
        b = (np.arange(E) % 5).astype(np.float32) * 0.25
    else:
        b = b.copy()
        b[[3, 77, 150]] = 50.0  # three tied winners with identical huge bias
        b[[10, 11]] = 40.0
    L.set_router(nw, rt, b)
    cpu = O.SynthLayer(C.WEIGHT_SEED)
    cpu.router, cpu.bias = np.ascontiguousarray(rt.ravel()), b
    x = C.inputs(0xC1, T)
    _, ids, wpre, _ = run(torch, L, x)
    L.close()
    r = cpu.route(x)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32))


@pytest.mark.parametrize("T", [1, 7, 64, 200, 400])
def test_expert_paths_match_oracle(torch, layer, cpu, T):
    """Every expert path (0 automatic, 1 wavefront GEMV, 2 MFMA grouped GEMM,
    3 / 4 its narrow / wide tile shape, 5 its 128-token tiles) meets the tolerance on the same
    tokens; routing is identical on all; hy3x_layer_last_path reports the
    path that ran (automatic: decode kernels at T = 1, the narrow MFMA shape
    below 320 tokens, the wide one from there, 128-token tiles from 1152)."""
    x = C.inputs(0xC2, T, first_token=300)
    rows = np.linspace(0, T - 1, min(T, 6)).astype(int)
    yo, ro = cpu.forward(x[rows])
    mfma_auto = 5 if T >= 1152 else 4 if T >= 320 else 3
    ran = {0: 0 if T == 1 else mfma_auto, 1: 1, 2: mfma_auto, 3: 3, 4: 4, 5: 5}
    try:
        for path in (0, 1, 2, 3, 4, 5):
            layer.set_path(path)
            y, ids, _, _ = run(torch, layer, x)
            assert layer.last_path() == ran[path], path
            assert np.array_equal(ids[rows], ro["ids"]), path
            assert O.rel_l2(y[rows] - x[rows], yo - x[rows]) <= TOL, path
    finally:
        layer.set_path(0)


@pytest.mark.parametrize("T,bad", [(1, np.nan), (3, np.nan), (40, np.nan), (40, np.inf)])
def test_non_finite_token(torch, layer, cpu, T, bad):
    """A token with a NaN or an infinity in x: its scores are NaN, and the
    selection with strict '>' (hy3.c:654-666) then keeps the experts in
    position order -- the routing equals the oracle's, with NaN gate weights
    and a NaN output row; every other token of the batch is bit for bit what
    it is without the bad token (decode path at T = 1, tiles otherwise)."""
    x = C.inputs(0xC8, T)
    bt = T // 2
    xb = x.copy()
    xb[bt, 5] = bad
    y, ids, wpre, w = run(torch, layer, xb)
    r = cpu.route(xb)
    assert np.array_equal(ids, r["ids"])
    assert np.isnan(wpre[bt]).all() and np.isnan(r["wpre"][bt]).all()
    ok = np.arange(T) != bt
    assert np.array_equal(wpre[ok].view(np.uint32), r["wpre"][ok].view(np.uint32))
    assert np.isnan(y[bt]).all()
    if T > 1:
        y0 = run(torch, layer, x)[0]
        assert np.array_equal(y[ok].view(np.uint32), y0[ok].view(np.uint32))


@pytest.mark.parametrize("T", [1, 2, 40, 300])
def test_non_finite_bias(torch, layer, cpu, T):
    """NaN and infinite router biases make some experts' scores non-finite
    while their sigmoids stay finite: a NaN taken at the scan's first position
    (experts 0 and 3 sit at the first positions) stays selected, NaNs
    elsewhere never win, +inf experts come first and -inf ones never (hy3.c
    :654-666). Routing equals the oracle's bit for bit, on every path, and the
    output is within the oracle's tolerance."""
    nw, rt, b0 = C.layer_small_tensors(C.WEIGHT_SEED)
    b = b0.copy()
    b[[0, 3, 64, 100, 150, 191]] = np.nan
    b[[7, 120]] = np.inf
    b[[1, 2, 5]] = -np.inf
    layer.set_router(nw, rt, b)
    saved = cpu.bias
    cpu.bias = b
    x = C.inputs(0xC9, T)
    try:
        r = cpu.route(x)
        assert set(r["ids"][:, :2].ravel().tolist()) <= {0, 7, 120}
        for path in ((0,) if T == 1 else (0, 3, 4, 5)):
            layer.set_path(path)
            y, ids, wpre, _ = run(torch, layer, x)
            assert np.array_equal(ids, r["ids"]), path
            assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32)), path
            assert np.isfinite(y).all()
        rows = np.linspace(0, T - 1, min(T, 4)).astype(int)
        yo, _ = cpu.forward(x[rows])
        assert O.rel_l2(y[rows] - x[rows], yo - x[rows]) <= TOL
    finally:
        layer.set_path(0)
        layer.set_router(nw, rt, b0)
        cpu.bias = saved


@pytest.mark.parametrize("T", [2, 40, 333, 1000, 1200, 4096])
def test_big_tiles_equal_narrow_tiles(torch, layer, cpu, T):
    """The 128-token tiles (activations staged per half block column, the
    dequantised weights reused over up to eight 16-token groups) do per
    element exactly the narrow tiles' arithmetic: the same output bit for bit,
    on tiles of every size class (1 to 8 token groups)."""
    x = C.inputs(0xC7, T)
    try:
        layer.set_path(3)
        y3, ids3, _, _ = run(torch, layer, x)
        layer.set_path(5)
        y5, ids5, _, _ = run(torch, layer, x)
        assert layer.last_path() == 5
    finally:
        layer.set_path(0)
    assert np.array_equal(ids3, ids5)
    assert np.array_equal(y3.view(np.uint32), y5.view(np.uint32))


@pytest.mark.parametrize("T", [16, 40, 64, 128, 129, 200, 257])
def test_mfma_tile_shapes_on_crowded_experts(torch, layer, cpu, T):
    """A bias of +50 on eight experts sends every token to them, so each of
    those experts holds all T tokens: the narrow shape (32-token tiles), the
    wide one (64-token tiles: T = 40 is one tile of 40 tokens, three 16-token
    column groups; T = 200 is three full tiles of four groups and one of 8
    tokens) and the 128-token tiles (T = 129 and 257: full tiles plus a tile of
    one token; T = 16, 64 and 128: tiles that end exactly on a 16-token column
    group) give the same output bit for bit (the same per-element arithmetic
    in every 16-token group and either shape), within the tolerance of the
    oracle's."""
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    hot = np.array([5, 17, 60, 61, 99, 130, 171, 191])
    b = b.copy()
    b[hot] = 50.0
    layer.set_router(nw, rt, b)
    saved = cpu.bias
    cpu.bias = b
    x = C.inputs(0xC5, T)
    try:
        out = {}
        for path in (3, 4, 5):
            layer.set_path(path)
            out[path], ids, _, _ = run(torch, layer, x)
            assert np.array_equal(np.sort(ids, axis=1), np.tile(np.sort(hot), (T, 1)))
        assert np.array_equal(out[3].view(np.uint32), out[4].view(np.uint32))
        assert np.array_equal(out[3].view(np.uint32), out[5].view(np.uint32))
        rows = np.linspace(0, T - 1, 5).astype(int)
        yo, _ = cpu.forward(x[rows])
        assert O.rel_l2(out[4][rows] - x[rows], yo - x[rows]) <= TOL
    finally:
        layer.set_path(0)
        layer.set_router(nw, rt, C.layer_small_tensors(C.WEIGHT_SEED)[2])
        cpu.bias = saved


@pytest.mark.parametrize("T", [1, 64, 400, 2100])
def test_graph_replay_matches_eager(torch, layer, T):
    """The forward only enqueues kernels, so it can be captured in a HIP graph
    (as the engine captures its decode step). Every replay -- with eager work
    and other forwards on the same layer in between -- reproduces the eager
    result bit for bit, on the decode kernels and the narrow, wide and
    128-token tiles."""
    x0 = torch.from_numpy(C.inputs(0xC2, T).copy()).cuda()
    xe = x0.clone()
    layer.forward(xe.data_ptr(), T, 8)
    torch.cuda.synchronize()
    y_eager = xe.cpu().numpy()
    xs = x0.clone()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            layer.forward(xs.data_ptr(), T, 8, stream=side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    other = torch.from_numpy(C.inputs(0xC1, T).copy()).cuda()
    for rep in range(4):
        xs.copy_(x0)
        _ = (other @ other.T).sum()  # unrelated eager work
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(xs.cpu().numpy().view(np.uint32), y_eager.view(np.uint32)), rep
        ot = other.clone()  # an eager forward on another buffer between replays
        layer.forward(ot.data_ptr(), T, 8)
        torch.cuda.synchronize()


# ------------------------------------------------------- hy3 Q8_0 shared expert
def test_q8_quantiser_matches_oracle(torch):
    """The device Q8_0 quantiser reproduces the oracle's bytes, which reproduce
    the reference converter's (tests/golden/q8_quant.npz)."""
    f = np.load(os.path.join(G, "q8_quant.npz"))
    x = torch.from_numpy(f["x"].ravel().copy()).cuda()
    out = torch.zeros(x.numel() // 32 * 36, dtype=torch.uint8, device="cuda")
    H._check(H.lib().hy3x_synth_quantize_q8_0(x.data_ptr(), out.data_ptr(), x.numel(), None))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), f["q"])


@pytest.fixture(scope="module")
def q8_mats():
    return tuple(O.gen_matrix_q8(C.WEIGHT_SEED, 0, k, E) for k in (O.T_GATE, O.T_UP, O.T_DOWN))


def q8_oracle(cpu, q8_mats, ids):
    """Oracle layer: the device's routed experts, the Q8_0 shared expert."""
    o = O.SynthLayer(C.WEIGHT_SEED, shared_q8=True)
    o.bias, o.has_bias = cpu.bias, cpu.has_bias
    for e in np.unique(ids):
        o.experts[int(e)] = cpu.expert(int(e))
    o.experts[E] = q8_mats
    return o


@pytest.fixture
def q8_layer(layer, cpu, q8_mats):
    set_bias(layer, cpu, "uniform")
    layer.set_shared_q8_0(*q8_mats)
    yield layer
    layer.set_expert_q4k(E, *cpu.expert(E))  # back to the Q4_K shared expert


def test_q8_shared_decode_matches_oracle_and_reference(torch, q8_layer, cpu, q8_mats):
    """T = 1 with hy3's Q8_0 shared expert: routing bit-exact, output within
    TOL of the oracle and of hy3.c's forward_layer_moe (moe_q8.npz)."""
    f = np.load(os.path.join(G, "moe_q8.npz"))
    x = O.normal(D, O.key(0xC0, 0, O.T_X), 1.0).reshape(1, D)
    y, ids, wpre, w = run(torch, q8_layer, x)
    yo, ro = q8_oracle(cpu, q8_mats, ids).forward(x)
    assert np.array_equal(ids, ro["ids"])
    assert np.array_equal(wpre.view(np.uint32), ro["wpre"].view(np.uint32))
    assert O.rel_l2(y - x, yo - x) <= TOL
    assert O.rel_l2(y - x, f["c0/y"] - x) <= TOL
    assert O.rel_l2(y, f["c0/y"]) <= TOL


def test_q8_shared_synth_equals_upload(torch, q8_layer):
    """hy3x_synth_shared_q8_0 (device generator + quantiser) gives the layer the
    same bytes as uploading the oracle's: identical outputs."""
    x = O.normal(D, O.key(0xC0, 0, O.T_X), 1.0).reshape(1, D)
    y1 = run(torch, q8_layer, x)[0]
    q8_layer.synth_shared_q8_0(C.WEIGHT_SEED, 0)
    y2 = run(torch, q8_layer, x)[0]
    assert np.array_equal(y1, y2)


def test_q4k_shared_restored_after_q8(torch, layer, cpu):
    """Setting expert 192 in Q4_K switches the layer back from the Q8 shared expert."""
    set_bias(layer, cpu, "uniform")
    x = O.normal(D, O.key(0xC0, 0, O.T_X), 1.0).reshape(1, D)
    y, ids, _, _ = run(torch, layer, x)
    yo, _ = cpu.forward(x)
    assert O.rel_l2(y - x, yo - x) <= TOL


@pytest.mark.parametrize("T,path", [(2, 0), (40, 3), (40, 4), (64, 4), (40, 5), (128, 5)])
def test_q8_shared_mfma_matches_oracle(torch, q8_layer, cpu, q8_mats, T, path):
    """T >= 2 with hy3's Q8_0 shared expert: the MFMA grouped GEMM runs the
    shared expert's tiles from its Q8 matrices (T = 40, narrow shape: one tile
    of 32 tokens and one of 8; wide shape: one tile of 40, three 16-token
    column groups; T = 64: one full wide tile; 128-token tiles: one tile of 40,
    one full tile of 128)."""
    x = O.normal(T * D, O.key(0xC1, 0, O.T_X), 1.0).reshape(T, D)
    q8_layer.set_path(path)
    try:
        y, ids, wpre, w = run(torch, q8_layer, x)
    finally:
        q8_layer.set_path(0)
    yo, ro = q8_oracle(cpu, q8_mats, ids).forward(x)
    assert np.array_equal(ids, ro["ids"])
    assert O.rel_l2(y - x, yo - x) <= TOL
    for t in range(T):
        assert O.rel_l2(y[t] - x[t], yo[t] - x[t]) <= 2 * TOL, t


@pytest.mark.parametrize("T", [40, 333, 2100])
def test_q8_shared_big_tiles_equal_narrow_tiles(torch, q8_layer, T):
    """With the Q8_0 shared expert the 128-token tiles run its tiles from the Q8
    matrices with the narrow tiles' arithmetic: the same output bit for bit
    (T = 2100 also runs them by default)."""
    x = O.normal(T * D, O.key(0xC6, 0, O.T_X), 1.0).reshape(T, D)
    try:
        q8_layer.set_path(3)
        y3 = run(torch, q8_layer, x)[0]
        q8_layer.set_path(5)
        y5 = run(torch, q8_layer, x)[0]
        assert q8_layer.last_path() == 5
        q8_layer.set_path(0)
        y0 = run(torch, q8_layer, x)[0]
        assert q8_layer.last_path() == (5 if T >= 1152 else 4 if T >= 320 else 3)
    finally:
        q8_layer.set_path(0)
    assert np.array_equal(y3.view(np.uint32), y5.view(np.uint32))
    assert np.array_equal(y3.view(np.uint32), y0.view(np.uint32))


def test_q8_shared_reference_tokens(torch, q8_layer):
    """hy3.c's forward_layer_moe with the Q8_0 shared expert on three config-1
    tokens (moe_q8.npz), through the batched (MFMA) path."""
    f = np.load(os.path.join(G, "moe_q8.npz"))
    y_ref = f["c1/y"]
    x = O.normal(y_ref.size, O.key(0xC1, 0, O.T_X), 1.0).reshape(y_ref.shape)
    y = run(torch, q8_layer, x)[0]
    assert O.rel_l2(y - x, y_ref - x) <= TOL


def test_q8_shared_gemv_path_is_refused(torch, q8_layer):
    """The GEMV tile path has no Q8 kernels: forcing it fails loudly."""
    x = O.normal(2 * D, O.key(0xC1, 0, O.T_X), 1.0).reshape(2, D)
    q8_layer.set_path(1)
    try:
        with pytest.raises(H.HY3XError):
            run(torch, q8_layer, x)
    finally:
        q8_layer.set_path(0)


@pytest.mark.parametrize("T", [1, 40, 300, 400])
def test_forward_residual_equals_add_then_forward(torch, layer, cpu, T):
    """hy3x_layer_forward_residual(x, a) == hy3x_layer_forward(x + a) bit for bit
    (every reader forms the same fp32 x + a), a is left unchanged, and the
    result matches the oracle on x + a."""
    set_bias(layer, cpu, "uniform")
    x = O.normal(T * D, O.key(0xC1, 0, O.T_X), 1.0).reshape(T, D)
    a = (O.normal(T * D, O.key(0xC2, 0, O.T_X), 1.0) * np.float32(0.5)).reshape(T, D)
    xd = torch.from_numpy(x.copy()).cuda()
    ad = torch.from_numpy(a.copy()).cuda()
    layer.forward_residual(xd.data_ptr(), ad.data_ptr(), T)
    torch.cuda.synchronize()
    y1 = xd.cpu().numpy()
    assert np.array_equal(ad.cpu().numpy(), a)
    xa = (x + a).astype(np.float32)
    y2 = run(torch, layer, xa)[0]
    assert np.array_equal(y1, y2)
    if T == 1:
        yo, _ = cpu.forward(xa)
        assert O.rel_l2(y1 - xa, yo - xa) <= TOL


def test_forward_residual_rejects_alias(torch, layer):
    xd = torch.zeros(D, dtype=torch.float32, device="cuda")
    with pytest.raises(H.HY3XError):
        layer.forward_residual(xd.data_ptr(), xd.data_ptr(), 1)


GGUF_IL = 1  # the first MoE layer (hy3.h: HY3_N_LAYER_DENSE = 1)


@pytest.fixture(scope="module")
def layer_gguf(cpu, q8_mats, tmp_path_factory):
    """The test layer written as a hy3 GGUF file with the converter's framing,
    tensor names and types (Q4_K routed experts, Q8_0 shared expert, F32
    router, norm and bias) at layer GGUF_IL, plus what the engine's loader
    requires of a whole model (hy3.c:889-898: token_embd.weight of [120832,
    4096], output.weight) and layer GGUF_IL's attention weights, all zero and
    written sparsely: zero Q8_0 blocks make the attention half add exactly
    +0 in hy3.c's forward_layer_moe (hy3.c:1226-1262)."""
    import sys
    sys.path.insert(0, G)
    from gguf_write import write_gguf
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    il = GGUF_IL
    t = [("token_embd.weight", 1, [120832, D], None),
         ("output_norm.weight", 0, [D], None),
         ("output.weight", 8, [120832, D], None),
         (f"blk.{il}.attn_norm.weight", 0, [D], None),
         (f"blk.{il}.attn_q.weight", 8, [64 * 128, D], None),
         (f"blk.{il}.attn_k.weight", 8, [8 * 128, D], None),
         (f"blk.{il}.attn_v.weight", 8, [8 * 128, D], None),
         (f"blk.{il}.attn_output.weight", 8, [D, 64 * 128], None),
         (f"blk.{il}.ffn_norm.weight", 0, [D], nw.view(np.uint8)),
         (f"blk.{il}.ffn_gate_inp.weight", 0, [E, D], rt.view(np.uint8)),
         (f"blk.{il}.ffn_gate_exps_b.bias", 0, [E], b.view(np.uint8))]
    kinds = ("gate", "up", "down")
    for e in range(E):
        for m, kind in enumerate(kinds):
            dims = [D, 1536] if kind == "down" else [1536, D]
            t.append((f"blk.{il}.ffn_{kind}_exps.{e}.{kind}_proj.weight", 12, dims,
                      cpu.expert(e)[m]))
    for m, kind in enumerate(kinds):
        dims = [D, 1536] if kind == "down" else [1536, D]
        t.append((f"blk.{il}.ffn_{kind}_shexp.weight", 8, dims, q8_mats[m]))
    path = tmp_path_factory.mktemp("gguf") / "hy3_layer.gguf"
    write_gguf(path, t)
    yield path
    path.unlink()


def test_load_gguf_layer_matches_source(torch, q8_layer, layer_gguf):
    """A whole layer loaded from a hy3 GGUF file by hy3x_layer_load_gguf
    computes exactly what the layer it came from computes (T = 1 and T = 40)."""
    assert H.gguf_check_layer(layer_gguf, GGUF_IL) == 8
    L2 = H.MoELayer(64)
    try:
        L2.load_gguf(layer_gguf, GGUF_IL)
        for T in (1, 40):
            x = O.normal(T * D, O.key(0xC2, 0, O.T_X), 1.0).reshape(T, D)
            y1 = run(torch, q8_layer, x)[0]
            y2 = run(torch, L2, x)[0]
            assert np.array_equal(y1, y2), T
    finally:
        L2.close()


REF_LIB = os.path.join(os.path.dirname(G), "..", "oracle", "_ref", "libhy3ref.so")
ENGINE_LIB = os.path.join(os.path.dirname(G), "..", "hy3_amd", "engine", "_build",
                          "libhy3gpu_moe.so")


@pytest.mark.skipif(not (os.path.exists(REF_LIB) and os.path.exists(ENGINE_LIB)),
                    reason="needs oracle/_ref and the engine drop-in (built where the "
                           "reference sources are present)")
@pytest.mark.parametrize("K", [8, 4])
def test_engine_loader_drop_in_matches_reference(torch, q8_layer, layer_gguf, K):
    """End to end through the engine's own objects: the file is loaded by
    hy3.c's hy3_model_load (hy3.c:805), the GPU drop-in is initialised from
    that hy3_model by hy3_gpu_init and run by hy3_gpu_ffn_moe_host, and
    hy3.c's forward_layer_moe runs on the same hy3_model on the host. The
    drop-in equals the library layer bit for bit (it bound the very tensors
    the loader mapped, with n_expert_used = K as HY3_TOP_K_EXPERTS sets it),
    and is within TOL of the reference, with the reference's top-K experts
    (from its recorded router scores, hy3.c:1272-1282) equal to the layer's."""
    import ctypes
    ref = ctypes.CDLL(REF_LIB)
    ref.hy3ref_model_load.restype = ctypes.c_void_p
    ref.hy3ref_model_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
    ref.hy3ref_model_moe.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_void_p]
    ref.hy3ref_model_n_expert_used.argtypes = [ctypes.c_void_p]
    ref.hy3ref_model_free.argtypes = [ctypes.c_void_p]
    eng = ctypes.CDLL(ENGINE_LIB)
    eng.hy3_gpu_init.argtypes = [ctypes.c_void_p, ctypes.c_int]
    eng.hy3_gpu_free.argtypes = [ctypes.c_void_p]
    eng.hy3_gpu_ffn_moe_host.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_int]
    m = ref.hy3ref_model_load(str(layer_gguf).encode(), 16, K)
    assert m
    try:
        assert ref.hy3ref_model_n_expert_used(m) == K
        assert eng.hy3_gpu_init(m, GGUF_IL + 1) == 0
        for T, seed in ((1, 0xE1), (5, 0xE2), (24, 0xE3)):
            x = O.normal(T * D, O.key(seed, 0, O.T_X), 1.0).reshape(T, D)
            y_gpu = np.ascontiguousarray(x.copy())
            assert eng.hy3_gpu_ffn_moe_host(m, GGUF_IL, y_gpu.ctypes.data, T) == 0
            y_lib, ids, _, _ = run(torch, q8_layer, x, K)
            assert np.array_equal(y_gpu.view(np.uint32), y_lib.view(np.uint32)), T
            y_ref = np.ascontiguousarray(x.copy())
            scores = np.zeros((T, E), np.float32)
            assert ref.hy3ref_model_moe(m, GGUF_IL, y_ref.ctypes.data, T,
                                        scores.ctypes.data) == 0
            ids_ref = np.argsort(-scores, axis=1, kind="stable")[:, :K]
            assert np.array_equal(np.sort(ids, 1), np.sort(ids_ref, 1)), T
            assert O.rel_l2(y_gpu - x, y_ref - x) <= TOL, T
    finally:
        eng.hy3_gpu_free(m)
        ref.hy3ref_model_free(m)
