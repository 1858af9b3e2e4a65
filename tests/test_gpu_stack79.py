"""Config 4 at its real depth: 79 stacked Hy3 MoE blocks (seed 0xC4, layer l),
about 162 GB of Q4_K resident in one MI355X's HBM, one token decoded through
all of them. Every layer's routing is checked bit-exact against the oracle
(ids identical, pre-scale weights bit-identical; hy3.c:1266-1291 per layer),
on the layer's actual input: the GPU's output of the layer before feeds both
sides. The output of a spread of layers is checked against the oracle's MoE
block within TOL (relative L2 on the delta and on y). Needs an MI355X: marked
gpu."""
import time

import numpy as np
import pytest

import hy3_amd as H
from hy3_amd import configs as C
from hy3_amd import hipmem
from oracle import hy3_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-3
N_LAYERS = 79
OUTPUT_CHECKED = (0, 1, 26, 52, 77, 78)


class DeviceBackedLayer(O.SynthLayer):
    """Oracle layer whose expert bytes are copied from the device arena."""

    def __init__(self, dev_layer, seed, layer):
        super().__init__(seed, layer)
        self.dev = dev_layer

    def expert(self, e):
        if e not in self.experts:
            self.experts[e] = tuple(hipmem.to_host(self.dev.expert_ptr(e, m), H.Q4K_MATRIX_BYTES)
                                    for m in range(3))
        return self.experts[e]


def test_stack79_routing_per_layer():
    import torch
    assert torch.cuda.is_available(), "no GPU"
    cfg = C.CONFIGS[4]
    assert cfg.n_layers == N_LAYERS
    t0 = time.time()
    layers = []
    try:
        for li in range(N_LAYERS):
            L = H.MoELayer(1)
            layers.append(L)
            L.synth_experts(cfg.weight_seed, li)
            nw, rt, b = C.layer_small_tensors(cfg.weight_seed, li)
            L.set_router(nw, rt, b)
        print(f"79 layers resident after {time.time() - t0:.1f} s", flush=True)
        x = C.inputs(cfg.input_seed, 1)
        xd = torch.from_numpy(x.copy()).cuda()
        for li, L in enumerate(layers):
            xin = xd.cpu().numpy()
            L.forward(xd.data_ptr(), 1)
            ids, wpre, _ = L.last_routing(1, 8)
            cpu = DeviceBackedLayer(L, cfg.weight_seed, li)
            r = cpu.route(xin)
            assert np.array_equal(ids, r["ids"]), li
            assert np.array_equal(wpre.view(np.uint32), r["wpre"].view(np.uint32)), li
            if li in OUTPUT_CHECKED:
                y = xd.cpu().numpy()
                yo, ro = cpu.forward(xin)
                assert np.array_equal(ro["ids"], ids), li
                assert O.rel_l2(y - xin, yo - xin) <= TOL, li
                assert O.rel_l2(y, yo) <= TOL, li
        y = xd.cpu().numpy()
        assert np.isfinite(y).all()
        print(f"79 layers checked after {time.time() - t0:.1f} s", flush=True)
    finally:
        for L in layers:
            L.close()
