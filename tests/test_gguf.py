"""GGUF-backed layer upload, CPU side: the test writer's framing against a file
the reference converter wrote, and the library's parser / layer check
(hy3x_gguf_check_layer, host code, no GPU) on full-size layer files and on
malformed ones."""
import os
import sys

import numpy as np
import pytest

import hy3_amd as H

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, G)
from gguf_read import Reader  # noqa: E402
from gguf_write import write_gguf  # noqa: E402

D, F, E = 4096, 1536, 192
SMALL = os.path.join(G, "convert_small.gguf")


def test_writer_matches_converter_framing(tmp_path):
    """Same tensors, same bytes: the writer reproduces the converter's file
    (header, key/values, tensor infos, alignment padding) exactly."""
    g = Reader(SMALL)
    assert g.version == 3 and g.kv["general.alignment"] == 32
    tensors = [(n, ty, dims, g.tensor_bytes(n)[0]) for n, (dims, ty, _) in g.tensors.items()]
    out = tmp_path / "w.gguf"
    write_gguf(out, tensors)
    assert out.read_bytes() == open(SMALL, "rb").read()


def layer_tensors(il, shared_type=8, bias=True):
    t = [(f"blk.{il}.ffn_norm.weight", 0, [D], None),
         (f"blk.{il}.ffn_gate_inp.weight", 0, [E, D], None)]
    if bias:
        t.append((f"blk.{il}.ffn_gate_exps_b.bias", 0, [E], None))
    for e in range(E):
        for kind in ("gate", "up", "down"):
            dims = [D, F] if kind == "down" else [F, D]
            t.append((f"blk.{il}.ffn_{kind}_exps.{e}.{kind}_proj.weight", 12, dims, None))
    for kind in ("gate", "up", "down"):
        dims = [D, F] if kind == "down" else [F, D]
        t.append((f"blk.{il}.ffn_{kind}_shexp.weight", shared_type, dims, None))
    return t


@pytest.mark.parametrize("shared_type", [8, 12])
def test_check_layer_full_size(tmp_path, shared_type):
    p = tmp_path / "layer.gguf"
    write_gguf(p, layer_tensors(5, shared_type))  # sparse: ~2 GB apparent, no data written
    assert H.gguf_check_layer(p, 5) == shared_type
    with pytest.raises(H.HY3XError, match=r"blk\.4\.ffn_norm\.weight not found"):
        H.gguf_check_layer(p, 4)


def test_check_layer_without_bias(tmp_path):
    p = tmp_path / "nobias.gguf"
    write_gguf(p, layer_tensors(2, 8, bias=False))
    assert H.gguf_check_layer(p, 2) == 8


def test_check_layer_names_the_bad_tensor(tmp_path):
    t = layer_tensors(1)
    missing = [x for x in t if x[0] != "blk.1.ffn_up_exps.77.up_proj.weight"]
    write_gguf(tmp_path / "a.gguf", missing)
    with pytest.raises(H.HY3XError, match=r"ffn_up_exps\.77\.up_proj\.weight not found"):
        H.gguf_check_layer(tmp_path / "a.gguf", 1)
    wrong = [(n, 8 if n == "blk.1.ffn_down_exps.3.down_proj.weight" else ty, d, v)
             for n, ty, d, v in t]
    write_gguf(tmp_path / "b.gguf", wrong)
    with pytest.raises(H.HY3XError, match=r"ffn_down_exps\.3\.down_proj\.weight: type 8"):
        H.gguf_check_layer(tmp_path / "b.gguf", 1)
    transposed = [(n, ty, [F, D] if n == "blk.1.ffn_down_exps.9.down_proj.weight" else d, v)
                  for n, ty, d, v in t]
    write_gguf(tmp_path / "c.gguf", transposed)
    with pytest.raises(H.HY3XError, match=r"down_proj\.weight: .*dim0 1536"):
        H.gguf_check_layer(tmp_path / "c.gguf", 1)


def test_check_layer_rejects_malformed_files(tmp_path):
    good = tmp_path / "g.gguf"
    write_gguf(good, layer_tensors(0))
    with open(good, "rb") as f:
        raw = f.read(4096)
        head = raw + f.read((1 << 20) - 4096)
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + (7).to_bytes(4, "little") + raw[8:],
        "truncated": raw[:200],
        "counts": raw[:8] + (1 << 40).to_bytes(8, "little") + raw[16:],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        with pytest.raises(H.HY3XError):
            H.gguf_check_layer(p, 0)
    # directory intact, data section cut short: a tensor extends past the end
    p = tmp_path / "short.gguf"
    p.write_bytes(head)
    with pytest.raises(H.HY3XError, match="past the end"):
        H.gguf_check_layer(p, 0)


def test_check_layer_on_converter_file():
    """The converter's own small file parses; its (small) tensors are reported
    with the shape mismatch rather than misread."""
    with pytest.raises(H.HY3XError, match=r"blk\.1\.ffn_norm\.weight: type 0, 256 elements"):
        H.gguf_check_layer(SMALL, 1)
