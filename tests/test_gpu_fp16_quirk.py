"""hy3.c's fp16 decode of the Q4_K block scales on the HIP path.

hy3.c's fp16_to_fp32 (hy3.c:354-369) maps every half with a zero exponent
(+-0 and the subnormals) to +-2^-15 * (1 + mantissa/1024) instead of the IEEE
value; dequantize_row_q4_K (hy3.c:1019-1043) applies it to d and dmin. The
HIP kernels reproduce it. Here blocks of the active experts get such d and
dmin values under their ordinary (non-zero) 6-bit scales, mins and quants, and
every expert path is checked against the oracle (which is pinned on all 65,536
halves against hy3.c). A contrast computed with IEEE halves shows that the
patched blocks move the output far beyond the tolerance, so a kernel with an
IEEE decode would fail this test. Needs an MI355X: marked gpu.
"""
import numpy as np
import pytest

import hy3_amd as H
from hy3_amd import configs as C
from hy3_amd import hipmem
from oracle import hy3_oracle as O

pytestmark = pytest.mark.gpu
D, F, E = 4096, 1536, 192
TOL = 1e-3
# zero-exponent halves: +0, -0, the smallest subnormal, mid and largest
# mantissas, and negative subnormals
QUIRK_HALVES = np.array([0x0000, 0x8000, 0x0001, 0x0200, 0x03FF, 0x8155, 0x0155], np.uint16)


def dequant_ieee(q):
    """Q4_K rows decoded with IEEE halves for d and dmin (the contrast)."""
    b = np.ascontiguousarray(q, np.uint8).reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.int32)
    sc = np.zeros((b.shape[0], 8), np.int32)
    mn = np.zeros((b.shape[0], 8), np.int32)
    for j in range(8):
        if j < 4:
            sc[:, j], mn[:, j] = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = b[:, 16:].astype(np.int32).reshape(-1, 4, 32)
    y = np.zeros((b.shape[0], 4, 2, 32), np.float32)
    for c in range(4):
        for hl, nib in ((0, qs[:, c] & 0xF), (1, qs[:, c] >> 4)):
            j = 2 * c + hl
            d1 = (d * sc[:, j].astype(np.float32)).astype(np.float32)
            m1 = (dm * mn[:, j].astype(np.float32)).astype(np.float32)
            y[:, c, hl] = d1[:, None] * nib.astype(np.float32) - m1[:, None]
    return y.reshape(-1)


def patch(q, salt):
    """Every other block gets zero-exponent d and dmin (scales and quants kept)."""
    b = np.ascontiguousarray(q, np.uint8).reshape(-1, 144).copy()
    idx = np.arange(0, b.shape[0], 2)
    dh = QUIRK_HALVES[(idx + salt) % QUIRK_HALVES.size]
    mh = QUIRK_HALVES[(idx + salt + 3) % QUIRK_HALVES.size]
    b[idx, 0:2] = dh.view(np.uint8).reshape(-1, 2)
    b[idx, 2:4] = mh.view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


def make_quirk_layer(T, seed):
    """A layer whose experts used by T test tokens carry quirk blocks, and its
    oracle twin holding the same bytes."""
    L = H.MoELayer(T)
    L.synth_experts(C.WEIGHT_SEED, 0)
    nw, rt, b = C.layer_small_tensors(C.WEIGHT_SEED)
    L.set_router(nw, rt, b)
    cpu = O.SynthLayer(C.WEIGHT_SEED)
    x = C.inputs(seed, T)
    used = set(cpu.route(x)["ids"].ravel().tolist()) | {E}
    for e in sorted(used):
        mats = [patch(hipmem.to_host(L.expert_ptr(e, m), H.Q4K_MATRIX_BYTES), e + m)
                for m in range(3)]
        L.set_expert_q4k(e, *mats)
        cpu.experts[e] = tuple(mats)
    return L, cpu, x


@pytest.fixture(scope="module")
def quirk_layer(torch):
    L, cpu, x = make_quirk_layer(8, 0xC8)
    yield L, cpu, x
    L.close()


@pytest.fixture(scope="module")
def quirk_layer_130(torch):
    """130 tokens: the 128-token tiles run a full token tile and a ragged one."""
    L, cpu, x = make_quirk_layer(130, 0xCA)
    yield L, cpu, x
    L.close()


def run_path(torch, L, cpu, xs, path):
    T = xs.shape[0]
    xd = torch.from_numpy(xs.copy()).cuda()
    L.set_path(path)
    try:
        L.forward(xd.data_ptr(), T)
        torch.cuda.synchronize()
        ids, wpre, _ = L.last_routing(T, 8)
    finally:
        L.set_path(0)
    y = xd.cpu().numpy()
    yo, ro = cpu.forward(xs)
    assert np.array_equal(ids, ro["ids"])
    assert np.array_equal(wpre.view(np.uint32), ro["wpre"].view(np.uint32))
    assert O.rel_l2(y - xs, yo - xs) <= TOL


def test_contrast_decoder_matches_oracle_on_normal_blocks():
    """The IEEE contrast decoder equals the oracle's decode where they agree by
    definition (normal d and dmin), so the contrast below is meaningful."""
    q = O.gen_matrix(C.WEIGHT_SEED, 0, O.T_GATE, 5)[: 144 * 64]
    assert np.array_equal(dequant_ieee(q).view(np.uint32), O.dequant(q).view(np.uint32))


def test_quirk_blocks_differ_from_ieee():
    q = patch(O.gen_matrix(C.WEIGHT_SEED, 0, O.T_UP, 7)[: 144 * 64], 0)
    a, b = O.dequant(q).reshape(-1, 256), dequant_ieee(q).reshape(-1, 256)
    assert np.array_equal(a[1::2], b[1::2])  # untouched blocks
    assert (a[0::2] != b[0::2]).any(axis=1).all()  # every patched block decodes differently


@pytest.mark.parametrize("T,path", [(1, 0), (8, 1), (8, 3), (8, 4), (8, 5), (1, 2)])
def test_quirk_blocks_on_every_path(torch, quirk_layer, T, path):
    """Decode kernels (T = 1), GEMV tiles, narrow, wide and 128-token MFMA
    tiles, and MFMA at T = 1: routing bit-exact, output within TOL of the
    oracle."""
    L, cpu, x = quirk_layer
    run_path(torch, L, cpu, x[:T], path)


@pytest.mark.parametrize("path", [4, 5])
def test_quirk_blocks_130_tokens(torch, quirk_layer_130, path):
    """130 tokens through the wide and the 128-token tiles (a full and a ragged
    token tile per hot expert)."""
    L, cpu, x = quirk_layer_130
    run_path(torch, L, cpu, x, path)


@pytest.mark.parametrize("T,path", [(1, 0), (8, 3), (8, 4), (8, 5)])
def test_quirk_blocks_with_q8_shared(torch, quirk_layer, T, path):
    """The routed experts' quirk blocks on the kernels' Q8_0-shared variants
    (hy3's real-checkpoint shared expert: the decode kernels and the narrow,
    wide and 128-token MFMA tiles with mfma_tile_q8): routing bit-exact, output
    within TOL of the oracle holding the same Q8_0 shared expert."""
    L, cpu, x = quirk_layer
    q8 = tuple(O.gen_matrix_q8(C.WEIGHT_SEED, 0, k, E) for k in (O.T_GATE, O.T_UP, O.T_DOWN))
    o = O.SynthLayer(C.WEIGHT_SEED, shared_q8=True)
    o.experts = {e: m for e, m in cpu.experts.items() if e != E}
    o.experts[E] = q8
    L.set_shared_q8_0(*q8)
    try:
        run_path(torch, L, o, x[:T], path)
    finally:
        L.set_expert_q4k(E, *cpu.experts[E])


def test_ieee_decode_would_fail(quirk_layer):
    """The same token with IEEE-decoded d/dmin lands far outside TOL of the
    oracle (hy3.c semantics): the path test above can tell the two apart."""
    _, cpu, x = quirk_layer
    x0 = x[:1]
    yo, ro = cpu.forward(x0)
    r = cpu.route(x0)
    s = r["s"][0].astype(np.float64)

    def ffn(e):
        g, u, dn = (dequant_ieee(m).astype(np.float64) for m in cpu.experts[e])
        gv, uv = g.reshape(F, D) @ s, u.reshape(F, D) @ s
        h = gv / (1.0 + np.exp(-gv)) * uv
        return dn.reshape(D, F) @ h

    delta = ffn(E) + sum(float(w) * ffn(int(e)) for e, w in zip(r["ids"][0], r["w"][0]))
    assert O.rel_l2(delta, (yo - x0)[0]) > 10 * TOL
