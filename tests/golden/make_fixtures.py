"""Write the golden fixtures from yuhai-china/hy3's own compiled code.

Runs ONLY in a container that holds the reference sources at /root/reference
(REF env var): builds oracle/_ref/libhy3ref.so from hy3.c and hy3_convert.c
(oracle/Makefile, target `ref`) and records what the reference computes:

  fp16_decode.npz   hy3.c fp16_to_fp32 (hy3.c:354-369) for all 65536 halves
  fp16_encode.npz   hy3_convert.c fp32_to_fp16 (hy3_convert.c:511-530) on edge inputs
  q4k_quant.npz     hy3_convert.c quantize_row_q4_K (:605-651) on edge + random blocks
  q4k_dequant.npz   hy3.c dequantize_row_q4_K (:1019-1043) on those blocks + special headers
  topk.npz          hy3.c topk_select (:654-666) on tie-heavy score vectors
  topk_nonfinite.npz  the same on score vectors holding NaN and +-inf
  layer.json        SHA-256 of every expert matrix of the synthetic layer (seed 0xC0,
                    layer 0) quantised by the reference quantiser, and of the small tensors
  moe.npz           hy3.c forward_layer_moe (:1219-1326) on config tokens: router scores
                    (sigmoid+bias), selected ids, sigmoid bits, output rows, and the
                    build's RMSNorm scale r per token (rsqrt estimate + Newton step,
                    host-CPU dependent), checked to reproduce forward_layer_moe's scores
  q8_quant.npz      hy3_convert.c's Q8_0 quantiser (:1192-1221, inline in the converter):
                    the converter run on a one-tensor safetensors directory holding edge
                    and random blocks as a shared-expert matrix (:684-697 force Q8_0),
                    and the Q8_0 bytes read back from the GGUF it writes
  moe_q8.npz        forward_layer_moe with the shared expert in hy3's Q8_0 (the type real
                    checkpoints carry), on config-0/1 tokens
  convert_small.gguf  the converter's output for a small safetensors directory holding one
                    MoE layer's tensor kinds (norm, router, bias, a routed expert, a shared
                    expert) at small shapes: the GGUF framing the writer and the library's
                    loader are checked against

Usage: python tests/golden/make_fixtures.py [--only q8|gguf|topk]   (all: about 2 minutes on 8 cores)
"""
import argparse
import hashlib
import json
import tempfile
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from oracle import hy3_oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("REF", "/root/reference")
E, D, F = 192, 4096, 1536


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def write_safetensors_dir(d, tensors):
    """model.safetensors.index.json + one F32 shard, the input hy3_convert reads
    (st_db_open, hy3_convert.c:246-410)."""
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, np.float32)
        header[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    hj = json.dumps(header).encode()
    hj += b" " * (-len(hj) % 8)
    shard = "model-00001-of-00001.safetensors"
    with open(os.path.join(d, shard), "wb") as f:
        f.write(len(hj).to_bytes(8, "little") + hj + b"".join(blobs))
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": {n: shard for n in tensors}}, f)


def q8_fixtures(R, lay_seed=0xC0):
    from gguf_read import Reader
    rng = np.random.default_rng(8)
    rows = []
    rows.append(np.zeros(256))
    rows.append(np.full(256, 0.5))
    rows.append(np.linspace(-1, 1, 256))
    r = np.arange(256) % 32 - 15.5; rows.append(r / 127.0 * 3.0)  # many exact halves of d
    rows.append(rng.standard_normal(256) * 1e-12)  # d floored at 1e-10
    rows.append(rng.standard_normal(256) * 1e4)
    r = rng.standard_normal(256) * 0.02; r[::32] = 0.5; rows.append(r)  # amax element -> 127
    r = rng.standard_normal(256) * 0.02; r[5::32] = -0.75; rows.append(r)  # negative amax -> -127
    r = np.round(rng.standard_normal(256) * 16) / 8; rows.append(r)
    for _ in range(23):
        rows.append(rng.standard_normal(256) * 0.02)
    x = np.stack(rows).astype(np.float32)  # [32 x 256]
    with tempfile.TemporaryDirectory() as d:
        write_safetensors_dir(d, {"model.layers.1.mlp.shared_mlp.gate_proj.weight": x})
        out = os.path.join(d, "q8.gguf")
        assert R.hy3ref_convert(d.encode(), out.encode(), 8) == 0
        g = Reader(out)
        q, dims, ty = g.tensor_bytes("blk.1.ffn_gate_shexp.weight")
    assert ty == 8 and q.size == x.size // 32 * 36, (ty, q.size)
    mine = O.quantize_q8(x.ravel())
    print(f"q8 quantiser: oracle-vs-reference byte mismatches {int((mine != q).sum())}", flush=True)
    np.savez_compressed(os.path.join(OUT, "q8_quant.npz"), x=x, q=q, dims=np.array(dims))

    # MoE block with a Q8_0 shared expert (every routed expert as in layer.json)
    lay = O.SynthLayer(lay_seed, shared_q8=True)
    fx = {}
    R.hy3ref_set_threads(os.cpu_count())
    for name, seed, nt in (("c0", 0xC0, 1), ("c1", 0xC1, 3)):
        x = O.normal(nt * D, O.key(seed, 0, O.T_X), 1.0).reshape(nt, D)
        y, scores = lay.ref_forward(x, 8)
        fx[f"{name}/x_seed"] = np.array([seed], np.int64)
        fx[f"{name}/scores"] = scores
        fx[f"{name}/y"] = y
        print(f"q8 case {name} done", flush=True)
    fx["shared_sha256"] = np.array([sha(m) for m in lay.expert(E)])
    np.savez_compressed(os.path.join(OUT, "moe_q8.npz"), **fx)


def gguf_fixture(R):
    rng = np.random.default_rng(9)
    t = {
        "model.layers.1.post_attention_layernorm.weight": rng.standard_normal(256),
        "model.layers.1.mlp.router.gate.weight": rng.standard_normal((4, 256)) * 0.02,
        "model.layers.1.mlp.expert_bias": rng.uniform(-0.1, 0.1, 4),
        "model.layers.1.mlp.experts.3.gate_proj.weight": rng.standard_normal((2, 256)) * 0.02,
        "model.layers.1.mlp.shared_mlp.down_proj.weight": rng.standard_normal((2, 64)) * 0.02,
    }
    with tempfile.TemporaryDirectory() as d:
        write_safetensors_dir(d, {k: np.asarray(v, np.float32) for k, v in t.items()})
        out = os.path.join(OUT, "convert_small.gguf")
        assert R.hy3ref_convert(d.encode(), out.encode(), 12) == 0
    print("gguf fixture written", flush=True)


def topk_nonfinite(R):
    """topk_nonfinite.npz: hy3.c topk_select (:654-666) on score vectors with
    NaN and +-inf entries (a NaN at the scan's first position is kept, a NaN
    elsewhere never wins)."""
    rng = np.random.default_rng(654)
    base = rng.standard_normal(192).astype(np.float32)
    sets = []
    s = np.full(192, np.nan, np.float32); sets.append(s)
    for where in (0, 1, 5, 7, 8, 191, int(np.argmax(base))):
        s = base.copy(); s[where] = np.nan; sets.append(s)
    s = base.copy(); s[::3] = np.nan; sets.append(s)
    s = base.copy(); s[1::2] = np.nan; sets.append(s)
    s = base.copy(); s[7] = np.inf; s[9] = -np.inf; s[100] = np.inf; sets.append(s)
    s = np.full(192, -np.inf, np.float32); sets.append(s)
    s = np.full(192, -np.inf, np.float32); s[50] = np.nan; s[2] = 0.0; sets.append(s)
    s = np.full(192, np.inf, np.float32); s[3] = np.nan; sets.append(s)
    s = np.full(192, np.nan, np.float32); s[[10, 70, 130]] = 1.0; sets.append(s)
    scores = np.stack(sets)
    vals = np.zeros((len(sets), 8, 8), np.float32)
    inds = np.full((len(sets), 8, 8), -1, np.int32)
    for i, sc in enumerate(scores):
        for k in range(1, 9):
            v = np.zeros(k, np.float32); ix = np.zeros(k, np.int32)
            R.hy3ref_topk_select(v.ctypes.data, ix.ctypes.data, sc.ctypes.data, 192, k)
            vals[i, k - 1, :k] = v; inds[i, k - 1, :k] = ix
    np.savez_compressed(os.path.join(OUT, "topk_nonfinite.npz"), scores=scores, vals=vals,
                        inds=inds)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=["q8", "gguf", "topk"], default=None)
    a = ap.parse_args()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref", f"REF={REF}"],
                   check=True)
    R = O.ref_lib()
    assert R is not None
    if a.only == "q8":
        q8_fixtures(R)
        return
    if a.only == "gguf":
        gguf_fixture(R)
        return
    if a.only == "topk":
        topk_nonfinite(R)
        return
    meta = {
        "reference": REF,
        "compiler": subprocess.run(["gcc", "--version"], capture_output=True,
                                   text=True).stdout.splitlines()[0],
        "flags": "-O3 -ffast-math -g -std=c99 -D_GNU_SOURCE -march=x86-64-v3 -fopenmp",
        "machine": platform.machine(),
        "generated": time.strftime("%Y-%m-%d"),
    }

    # fp16 decode, all halves
    h = np.arange(65536, dtype=np.uint32)
    dec = np.array([R.hy3ref_fp16_to_fp32(int(v)) for v in h], np.float32).view(np.uint32)
    np.savez_compressed(os.path.join(OUT, "fp16_decode.npz"), bits=dec)

    # fp16 encode on edge inputs
    rng = np.random.default_rng(11)
    edge = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 1e6, -1e6, 6.1035156e-05,
                     6.0e-05, 5.9604645e-08, 1e-8, 1e-40, -1e-40, np.inf, -np.inf, np.nan,
                     1.0009765625, 0.333333, 1.5e-5, 3.1e-5, 2.0**-14, 2.0**-15, 2.0**-24],
                    np.float32)
    enc_in = np.concatenate([edge, (rng.standard_normal(2000) * np.exp(
        rng.uniform(-20, 12, 2000))).astype(np.float32)])
    enc_out = np.array([R.hy3ref_fp32_to_fp16(float(v)) for v in enc_in], np.uint16)
    np.savez_compressed(os.path.join(OUT, "fp16_encode.npz"), x=enc_in, h=enc_out)

    # quantiser: edge blocks + random blocks
    blocks = []
    blocks.append(np.zeros(256))
    blocks.append(np.full(256, 0.5))
    blocks.append(np.full(256, -0.25))
    blocks.append(np.linspace(0, 1, 256))
    blocks.append(np.linspace(-1, 0, 256))
    blocks.append(np.linspace(-3, 3, 256))
    blocks.append(rng.standard_normal(256) * 1e-12)
    blocks.append(rng.standard_normal(256) * 1e-6)
    blocks.append(rng.standard_normal(256) * 1e4)
    b = rng.standard_normal(256) * 0.02; b[:32] = 0.0; blocks.append(b)
    b = np.abs(rng.standard_normal(256)) * 0.02; blocks.append(b)
    b = rng.standard_normal(256) * 0.02; b[7] = 5.0; blocks.append(b)
    b = np.round(rng.standard_normal(256) * 8) / 16; blocks.append(b)
    b = rng.standard_normal(256) * 0.002; blocks.append(b)
    for _ in range(16):
        blocks.append(rng.standard_normal(256) * 0.02)
    blocks.append(O.normal(256 * 64, O.key(0xC0, 0, O.T_GATE, 0), 0.02))
    qx = np.concatenate(blocks).astype(np.float32)
    qref = np.zeros(qx.size // 256 * 144, np.uint8)
    R.hy3ref_quantize_q4k(qx.ctypes.data, qref.ctypes.data, qx.size)
    np.savez_compressed(os.path.join(OUT, "q4k_quant.npz"), x=qx, q=qref)

    # dequantiser: the quantised blocks plus hand-built special headers
    special = []
    for dbits, mbits in [(0x0000, 0x0000), (0x0001, 0x03FF), (0x8000, 0x0001), (0x3C00, 0x3C00),
                         (0x0400, 0x0400), (0x7BFF, 0x0000), (0x03FF, 0x2000), (0x2E66, 0x1A00)]:
        blk = np.zeros(144, np.uint8)
        blk[0:2] = np.frombuffer(np.uint16(dbits).tobytes(), np.uint8)
        blk[2:4] = np.frombuffer(np.uint16(mbits).tobytes(), np.uint8)
        blk[4:16] = rng.integers(0, 256, 12, dtype=np.uint8)
        blk[16:] = rng.integers(0, 256, 128, dtype=np.uint8)
        special.append(blk)
    allones = np.full(144, 0xFF, np.uint8); allones[0:4] = [0x00, 0x3C, 0x00, 0x3C]
    special.append(allones)
    dq_in = np.concatenate([qref, np.concatenate(special)])
    dq_out = np.zeros(dq_in.size // 144 * 256, np.float32)
    R.hy3ref_dequant_q4k(dq_out.ctypes.data, dq_in.ctypes.data, dq_out.size)
    np.savez_compressed(os.path.join(OUT, "q4k_dequant.npz"), q=dq_in, y=dq_out)

    # top-k with ties
    sets = []
    sets.append(rng.standard_normal(192).astype(np.float32))
    s = np.zeros(192, np.float32); sets.append(s)
    s = np.round(rng.standard_normal(192) * 2).astype(np.float32); sets.append(s)
    s = np.full(192, 0.5, np.float32); s[[5, 77, 191]] = 0.7; s[[3, 100]] = 0.6; sets.append(s)
    s = np.round(rng.uniform(0, 4, 192)).astype(np.float32); s[::2] *= -1; sets.append(s)
    s = np.full(192, -0.0, np.float32); s[::3] = 0.0; sets.append(s)
    s = np.arange(192, dtype=np.float32)[::-1].copy(); sets.append(s)
    s = (np.arange(192) % 7).astype(np.float32); sets.append(s)
    for _ in range(8):
        sets.append(np.round(rng.uniform(0, 3, 192)).astype(np.float32))
    scores = np.stack(sets)
    vals = np.zeros((len(sets), 8, 8), np.float32)
    inds = np.full((len(sets), 8, 8), -1, np.int32)
    for i, sc in enumerate(scores):
        for k in range(1, 9):
            v = np.zeros(k, np.float32); ix = np.zeros(k, np.int32)
            R.hy3ref_topk_select(v.ctypes.data, ix.ctypes.data, sc.ctypes.data, 192, k)
            vals[i, k - 1, :k] = v; inds[i, k - 1, :k] = ix
    np.savez_compressed(os.path.join(OUT, "topk.npz"), scores=scores, vals=vals, inds=inds)
    topk_nonfinite(R)
    print("unit fixtures done", flush=True)

    # the synthetic layer, quantised by the reference quantiser
    t0 = time.time()
    lay = O.SynthLayer(0xC0)
    hashes = {}
    mismatch = 0
    for e in range(E + 1):
        mats = []
        for kind in (O.T_GATE, O.T_UP, O.T_DOWN):
            rows, cols = (D, F) if kind == O.T_DOWN else (F, D)
            x = O.normal(rows * cols, O.key(0xC0, 0, kind, e), 0.02)
            q = np.zeros(O.MAT_BYTES, np.uint8)
            R.hy3ref_quantize_q4k(x.ctypes.data, q.ctypes.data, x.size)
            mats.append(q)
        hashes[str(e)] = [sha(m) for m in mats]
        mine = lay.expert(e)
        mismatch += sum(int(not np.array_equal(a, b)) for a, b in zip(mats, mine))
        lay.experts[e] = tuple(mats)
    print(f"layer generated in {time.time() - t0:.1f}s; oracle-vs-reference matrix mismatches: "
          f"{mismatch}", flush=True)
    layer_meta = {
        "seed": 0xC0, "layer": 0, "expert_sha256": hashes,
        "norm_w_sha256": sha(lay.norm_w), "router_sha256": sha(lay.router),
        "bias_sha256": sha(lay.bias),
        "zipf_bias_0xC3_sha256": sha(O.zipf_bias(E, 0xC3)),
        "x_0xC0_t0_sha256": sha(O.normal(D, O.key(0xC0, 0, O.T_X), 1.0)),
        "oracle_quantiser_mismatches": mismatch, **meta,
    }
    with open(os.path.join(OUT, "layer.json"), "w") as f:
        json.dump(layer_meta, f, indent=1, sort_keys=True)

    # MoE block fixtures
    cases = [  # name, input seed, tokens routed, tokens with y, K, bias kind
        ("c0", 0xC0, 1, 1, 8, "uniform"),
        ("c0_k4", 0xC0, 1, 1, 4, "uniform"),
        ("c0_nobias", 0xC0, 1, 1, 8, "none"),
        ("c1", 0xC1, 32, 4, 8, "uniform"),
        ("c2", 0xC2, 64, 2, 8, "uniform"),
        ("c3", 0xC3, 64, 2, 8, "zipf"),
    ]
    fx = {}
    R.hy3ref_set_threads(os.cpu_count())
    uni_bias = lay.bias.copy()
    for name, seed, nt, ny, K, bk in cases:
        x = O.normal(nt * D, O.key(seed, 0, O.T_X), 1.0).reshape(nt, D)
        lay.bias = O.zipf_bias(E, seed) if bk == "zipf" else uni_bias
        lay.has_bias = bk != "none"
        y, scores = lay.ref_forward(x, K)
        lay.has_bias = False
        _, sig = lay.ref_forward(x, K)  # scores without bias are the sigmoid values
        lay.has_bias = True
        ids = np.zeros((nt, K), np.int32)
        rr = np.zeros(nt, np.float32)
        for t in range(nt):
            rr[t] = R.hy3ref_rms_r(x[t].ctypes.data, D)
            sv = np.zeros(D, np.float32); lg = np.zeros(E, np.float32); sc2 = np.zeros(E, np.float32)
            R.hy3ref_router_scores(x[t].ctypes.data, lay.norm_w.ctypes.data, lay.router.ctypes.data,
                                   lay.bias.ctypes.data, 0 if bk == "none" else 1, sv.ctypes.data,
                                   lg.ctypes.data, sc2.ctypes.data)
            assert np.array_equal(sc2.view(np.uint32), scores[t].view(np.uint32)), (name, t)
            v = np.zeros(K, np.float32); ix = np.zeros(K, np.int32)
            R.hy3ref_topk_select(v.ctypes.data, ix.ctypes.data, scores[t].ctypes.data, E, K)
            ids[t] = ix
        fx[f"{name}/x_seed"] = np.array([seed], np.int64)
        fx[f"{name}/K"] = np.array([K], np.int32)
        fx[f"{name}/bias_kind"] = np.array([bk])
        fx[f"{name}/scores"] = scores
        fx[f"{name}/sigmoid"] = sig
        fx[f"{name}/ids"] = ids
        fx[f"{name}/rms_r"] = rr
        fx[f"{name}/y"] = y[:ny]
        print(f"case {name} done", flush=True)
    lay.bias = uni_bias
    np.savez_compressed(os.path.join(OUT, "moe.npz"), **fx)
    q8_fixtures(R)
    gguf_fixture(R)
    print("all fixtures written", flush=True)


if __name__ == "__main__":
    main()
