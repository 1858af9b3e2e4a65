"""The CPU oracle against the reference's own compiled code (golden fixtures
written by tests/golden/make_fixtures.py from /root/reference) and against
closed forms. CPU only."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import hy3_oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E, D = 192, 4096


def load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def layer_meta():
    with open(os.path.join(G, "layer.json")) as f:
        return json.load(f)


def ulp_dist(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


# ---------------------------------------------------------------- fp16 / Q4_K
def test_fp16_decode_all_halves():
    ref = load("fp16_decode.npz")["bits"]
    got = np.array([O.lib().hy3o_fp16_to_fp32(h) for h in range(65536)], np.float32).view(np.uint32)
    assert np.array_equal(got, ref)


def test_fp16_decode_quirk_exp0():
    # hy3.c decodes exponent-0 halves as 2^-15 * (1 + m/1024), not as subnormals
    assert O.lib().hy3o_fp16_to_fp32(0x0000) == pytest.approx(2.0 ** -15, rel=0)
    assert O.lib().hy3o_fp16_to_fp32(0x8000) == -(2.0 ** -15)
    assert O.lib().hy3o_fp16_to_fp32(0x3C00) == 1.0
    assert O.lib().hy3o_fp16_to_fp32(0x7BFF) == 65504.0


def test_fp16_encode_truncating():
    f = load("fp16_encode.npz")
    got = np.array([O.lib().hy3o_fp32_to_fp16_trunc(float(v)) for v in f["x"]], np.uint16)
    assert np.array_equal(got, f["h"])


def test_quantizer_matches_reference():
    f = load("q4k_quant.npz")
    assert np.array_equal(O.quantize(f["x"]), f["q"])


def test_dequant_matches_reference():
    f = load("q4k_dequant.npz")
    assert np.array_equal(O.dequant(f["q"]).view(np.uint32), f["y"].view(np.uint32))


def test_dequant_closed_form():
    # d = 1.0, dmin = 0.5, every 6-bit scale 63 and min 0 -> w = 63*q
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x38]
    blk[4:8] = 63
    blk[8:12] = 0
    blk[12:16] = 0x0F | 0x00  # sub-blocks 4..7: scale low 4 bits 15, min 0
    blk[4:8] |= 0xC0          # scale high 2 bits for sub-blocks 4..7 (=3 -> 63)
    q = np.arange(128, dtype=np.uint8)
    blk[16:] = q
    y = O.dequant(blk)
    for c in range(4):
        lo = q[32 * c:32 * c + 32] & 0xF
        hi = q[32 * c:32 * c + 32] >> 4
        assert np.array_equal(y[64 * c:64 * c + 32], 63.0 * lo)
        assert np.array_equal(y[64 * c + 32:64 * c + 64], 63.0 * hi)


def test_quant_roundtrip_error_bound():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256 * 512) * 0.02).astype(np.float32)
    y = O.dequant(O.quantize(x))
    err = np.abs(y - x).reshape(-1, 32)
    span = (x.reshape(-1, 32).max(1) - x.reshape(-1, 32).min(1))
    # 4-bit levels over the sub-block span, with 6-bit scale/min rounding slack
    assert np.all(err.max(1) <= span / 15 * 0.75 + 1e-3)
    assert np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2)) < 0.15


# ---------------------------------------------------------------- routing
def test_topk_matches_reference():
    f = load("topk.npz")
    for i, sc in enumerate(f["scores"]):
        for k in range(1, 9):
            v, ix = O.topk_select(sc, k)
            assert np.array_equal(ix, f["inds"][i, k - 1, :k]), (i, k)
            assert np.array_equal(v.view(np.uint32), f["vals"][i, k - 1, :k].view(np.uint32))


def test_topk_nonfinite_matches_reference():
    # NaN / inf scores: a NaN at the scan's first position stays, others never win
    f = load("topk_nonfinite.npz")
    for i, sc in enumerate(f["scores"]):
        for k in range(1, 9):
            v, ix = O.topk_select(sc, k)
            assert np.array_equal(ix, f["inds"][i, k - 1, :k]), (i, k)
            assert np.array_equal(v.view(np.uint32), f["vals"][i, k - 1, :k].view(np.uint32))


def test_topk_invariants():
    rng = np.random.default_rng(5)
    for _ in range(50):
        sc = rng.standard_normal(192).astype(np.float32)
        v, ix = O.topk_select(sc, 8)
        assert len(set(ix.tolist())) == 8
        assert np.all(np.diff(v) <= 0)
        assert np.array_equal(np.sort(sc)[::-1][:8], v)
        sc2 = sc.copy(); sc2[17] = 100.0
        assert 17 in O.topk_select(sc2, 8)[1]


def test_sig_expf_accuracy():
    x = np.linspace(-87.0, 88.0, 400001).astype(np.float32)
    got = np.array([O.lib().hy3o_sig_expf(float(v)) for v in x[::7]], np.float32)
    ref = np.exp(x[::7].astype(np.float64)).astype(np.float32)
    assert ulp_dist(got, ref).max() <= 0


def test_dot8_vs_fp64():
    rng = np.random.default_rng(7)
    for _ in range(20):
        a = rng.standard_normal(4096).astype(np.float32)
        b = rng.standard_normal(4096).astype(np.float32)
        got = O.lib().hy3o_dot8(a.ctypes.data, b.ctypes.data, 4096)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = 4096 * 2.0 ** -24 * float(np.sum(np.abs(a.astype(np.float64) * b)))
        assert abs(got - exact) <= bound
    # exact on integer data (no rounding anywhere)
    a = np.arange(4096, dtype=np.float32) % 5
    b = np.ones(4096, np.float32)
    assert O.lib().hy3o_dot8(a.ctypes.data, b.ctypes.data, 4096) == float(a.sum())


def test_rms_norm_vs_fp64():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(4096).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    out = np.zeros(4096, np.float32)
    O.lib().hy3o_rms_norm(out.ctypes.data, x.ctypes.data, w.ctypes.data, 4096)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-5) * w
    assert np.max(np.abs(out - ref) / np.abs(ref).max()) < 1e-6


def test_route_weights_sum_to_scale():
    lay = O.SynthLayer(0xC0)
    x = O.normal(8 * D, O.key(0xC2, 0, O.T_X), 1.0).reshape(8, D)
    r = lay.route(x)
    np.testing.assert_allclose(r["w"].sum(1), 2.826, rtol=1e-6)
    np.testing.assert_allclose(r["wpre"].sum(1), 1.0, rtol=1e-6)


# ---------------------------------------------------------------- synthetic inputs
def test_small_tensors_match_spec(layer_meta):
    lay = O.SynthLayer(0xC0)
    assert sha(lay.norm_w) == layer_meta["norm_w_sha256"]
    assert sha(lay.router) == layer_meta["router_sha256"]
    assert sha(lay.bias) == layer_meta["bias_sha256"]
    assert sha(O.zipf_bias(E, 0xC3)) == layer_meta["zipf_bias_0xC3_sha256"]
    assert sha(O.normal(D, O.key(0xC0, 0, O.T_X), 1.0)) == layer_meta["x_0xC0_t0_sha256"]


@pytest.mark.parametrize("expert", [0, 131, 192])
def test_expert_bytes_match_reference_quantiser(layer_meta, expert):
    lay = O.SynthLayer(0xC0)
    got = [sha(m) for m in lay.expert(expert)]
    assert got == layer_meta["expert_sha256"][str(expert)]


# ---------------------------------------------------------------- MoE block vs hy3.c
MOE_CASES = ["c0", "c0_k4", "c0_nobias", "c1", "c2", "c3"]


@pytest.fixture(scope="module")
def moe():
    return load("moe.npz")


@pytest.fixture(scope="module")
def base_layer():
    return O.SynthLayer(0xC0)


def case_layer(base, moe, name):
    bk = str(moe[f"{name}/bias_kind"][0])
    if bk == "zipf":
        base.bias = O.zipf_bias(E, int(moe[f"{name}/x_seed"][0]))
    else:
        base.bias = O.uniform_sym(E, O.key(0xC0, 0, O.T_BIAS), 0.1)
    base.has_bias = bk != "none"
    return base


def ref_wpre(sig, ids):
    sel = sig[np.arange(ids.shape[0])[:, None], ids].astype(np.float32)
    s = np.zeros(ids.shape[0], np.float32)
    for k in range(ids.shape[1]):
        s = (s + sel[:, k]).astype(np.float32)
    inv = (np.float32(1.0) / (s + np.float32(1e-20))).astype(np.float32)
    return (sel * inv[:, None]).astype(np.float32)


def case_inputs(moe, name):
    ids_ref = moe[f"{name}/ids"]
    T = ids_ref.shape[0]
    x = O.normal(T * D, O.key(int(moe[f"{name}/x_seed"][0]), 0, O.T_X), 1.0).reshape(T, D)
    return x, ids_ref


@pytest.mark.parametrize("name", MOE_CASES)
def test_routing_matches_reference_given_its_rms_scale(moe, base_layer, name):
    """Fed the reference build's own RMSNorm scale r (its rsqrt estimate plus a
    Newton step, host-CPU dependent), the routing contract reproduces hy3.c:
    identical ids and pre-scale gate weights within 1 ulp; sigmoid within 2 ulp
    (glibc's scalar expf is not always correctly rounded; the contract's is)."""
    lay = case_layer(base_layer, moe, name)
    x, ids_ref = case_inputs(moe, name)
    r = lay.route(x, ids_ref.shape[1], r_override=moe[f"{name}/rms_r"])
    assert np.array_equal(r["ids"], ids_ref)
    u = ulp_dist(r["sigmoid"], moe[f"{name}/sigmoid"])
    assert u.max() <= 2 and np.mean(u == 0) > 0.99
    assert ulp_dist(r["wpre"], ref_wpre(moe[f"{name}/sigmoid"], ids_ref)).max() <= 1


@pytest.mark.parametrize("name", MOE_CASES)
def test_routing_matches_reference(moe, base_layer, name):
    """With the contract's correctly rounded r: identical ids; gate weights
    within a few ulp (the whole difference is the CPU's rsqrt estimate)."""
    lay = case_layer(base_layer, moe, name)
    x, ids_ref = case_inputs(moe, name)
    r = lay.route(x, ids_ref.shape[1])
    assert np.array_equal(r["ids"], ids_ref)
    r_ref = moe[f"{name}/rms_r"]
    assert ulp_dist(r["wpre"], ref_wpre(moe[f"{name}/sigmoid"], ids_ref)).max() <= 8
    np.testing.assert_allclose(r["sigmoid"], moe[f"{name}/sigmoid"], rtol=4e-6)
    assert np.all(r_ref > 0)


@pytest.mark.parametrize("name", MOE_CASES)
def test_block_output_matches_reference(moe, base_layer, name):
    lay = case_layer(base_layer, moe, name)
    y_ref = moe[f"{name}/y"]
    T, K = y_ref.shape[0], moe[f"{name}/ids"].shape[1]
    x = O.normal(T * D, O.key(int(moe[f"{name}/x_seed"][0]), 0, O.T_X), 1.0).reshape(T, D)
    y, r = lay.forward(x, K)
    assert np.array_equal(r["ids"], moe[f"{name}/ids"][:T])
    assert O.rel_l2(y - x, y_ref - x) < 1e-5
    assert O.rel_l2(y, y_ref) < 1e-5


# ------------------------------------------------------------ hy3 Q8_0 (shared)
def test_q8_quantizer_matches_reference():
    """hy3_convert.c's Q8_0 quantiser (inline in the converter, :1192-1221) as the
    reference build computes it: the fixture holds the bytes its converter wrote
    for edge and random blocks; the restatement reproduces every byte. 14 of the
    fixture's 256 blocks have an amax for which amax*(1/127) and amax/127 round
    differently, so the fast-math reciprocal form is pinned too."""
    f = load("q8_quant.npz")
    assert np.array_equal(O.quantize_q8(f["x"].ravel()), f["q"])
    amax = np.abs(f["x"].reshape(-1, 32)).max(1).astype(np.float32)
    assert np.sum(amax * np.float32(1.0 / 127.0) != amax / np.float32(127.0)) > 0


def test_q8_quant_properties():
    """Closed-form facts of the quantiser: |q| <= 127; the block's largest |x|
    maps to +-127 when d is not floored; |x - d q| <= d/2 (plus rounding of
    x/d); d >= 1e-10."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(32 * 64) * 0.02, rng.standard_normal(32 * 4) * 1e-13,
                        np.zeros(32)]).astype(np.float32)
    q = O.quantize_q8(x)
    blk = q.reshape(-1, 36)
    d = blk[:, :4].copy().view(np.float32)[:, 0]
    qs = blk[:, 4:].view(np.int8).astype(np.int32)
    xb = x.reshape(-1, 32)
    assert np.all(np.abs(qs) <= 127) and np.all(d >= np.float32(1e-10))
    big = d > 1e-10
    assert np.all(np.abs(qs[big]).max(1) == 127)
    err = np.abs(xb - d[:, None] * qs)
    assert np.all(err <= d[:, None] * 0.5 * (1 + 1e-5) + 1e-30)
    np.testing.assert_array_equal(O.dequant_q8(q), (d[:, None] * qs).astype(np.float32).ravel())


def test_q8_matvec_vs_fp64():
    """hy3.c:1098-1120 (one fp32 sum per row of d*q*x) against an fp64 brute
    force over the dequantised weights."""
    rng = np.random.default_rng(4)
    m, n = 48, 512
    w = O.quantize_q8((rng.standard_normal(m * n) * 0.02).astype(np.float32))
    x = rng.standard_normal(n).astype(np.float32)
    out = np.zeros(m, np.float32)
    O.lib().hy3o_mul_mat_q8_0(out.ctypes.data, w.ctypes.data, x.ctypes.data, m, n)
    ref = O.dequant_q8(w).reshape(m, n).astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    # a single nonzero weight picks out d * q * x exactly
    w2 = np.zeros(36 * (n // 32), np.uint8)
    w2[0:4] = np.frombuffer(np.float32(0.25).tobytes(), np.uint8)
    w2[4 + 7] = np.uint8(np.int8(-3).view(np.uint8))
    o2 = np.zeros(1, np.float32)
    O.lib().hy3o_mul_mat_q8_0(o2.ctypes.data, w2.ctypes.data, x.ctypes.data, 1, n)
    assert o2[0] == np.float32(0.25 * -3.0) * x[7]


@pytest.fixture(scope="module")
def q8_layer():
    return O.SynthLayer(0xC0, shared_q8=True)


def test_q8_shared_bytes_match_fixture(q8_layer):
    ref = [str(s) for s in load("moe_q8.npz")["shared_sha256"]]
    assert [sha(m) for m in q8_layer.expert(E)] == ref


@pytest.mark.parametrize("name", ["c0", "c1"])
def test_q8_block_output_matches_reference(q8_layer, name):
    """forward_layer_moe with hy3's Q8_0 shared expert (hy3.c:1293-1300,
    1322-1323 through mul_mat_f32 case 8): the oracle's block output."""
    f = load("moe_q8.npz")
    y_ref = f[f"{name}/y"]
    T = y_ref.shape[0]
    x = O.normal(T * D, O.key(int(f[f"{name}/x_seed"][0]), 0, O.T_X), 1.0).reshape(T, D)
    y, _ = q8_layer.forward(x, 8)
    assert O.rel_l2(y - x, y_ref - x) < 1e-5
