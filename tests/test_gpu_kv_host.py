"""The host-resident prefix cache (qimm_kv_create_host, the reference's
--kv-cache-cpu / set_kv_cache_offload, src/transformer.rs:26-45) gives the
same block outputs as the device cache, bit for bit: without prefetch (each
layer copied on use, src/transformer.rs:43-45), with prefetch of layer l+1 on a
separate copy stream while layer l computes, and with prefetches in irregular
order; loads return the stored bytes and a re-stored layer replaces its staged
copy. One oracle check anchors the cached step itself."""
import numpy as np
import pytest

import oracle as O
import qimm
import synth
from gpu_util import cos_sim, dev, host, max_abs_rel, stream
from test_gpu_block import SMALL, block_tensors, make_case

pytestmark = pytest.mark.gpu

L = 4


class Setup:
    def __init__(self, torch, qctx, seed, b=1, s=64, p=40):
        self.torch, self.qctx = torch, qctx
        self.w, self.x, self.mod, self.pe, _, _ = make_case(seed, SMALL, b, s, p, synth.Q4_K, synth.Q6_K)
        rng = np.random.default_rng(seed + 1)
        self.k = [O.f32_to_bf16(rng.standard_normal((b, SMALL["heads"], p, 128))) for _ in range(L)]
        self.v = [O.f32_to_bf16(rng.standard_normal((b, SMALL["heads"], p, 128))) for _ in range(L)]
        self.keep = []
        self.blk = qctx.block_create(qimm.BlockConfig(SMALL["hidden"], SMALL["heads"], 128, SMALL["mlp"]),
                                     block_tensors(self.w, self.keep))
        self.b, self.s, self.p = b, s, p
        self.x_d, self.mod_d, self.pe_d = dev(torch, self.x), dev(torch, self.mod), dev(torch, self.pe)
        self.out = torch.empty_like(self.x_d)

    def cache(self, host_cache):
        mk = self.qctx.kv_create_host if host_cache else self.qctx.kv_create
        kv = mk(L, self.b, SMALL["heads"], self.p)
        assert kv.is_host == host_cache
        for layer in range(L):
            self.store(kv, layer, self.k[layer], self.v[layer])
        return kv

    def store(self, kv, layer, k, v):
        k_d, v_d = dev(self.torch, k.view(np.int16)), dev(self.torch, v.view(np.int16))
        kv.store(layer, k_d.data_ptr(), v_d.data_ptr(), stream(self.torch))
        self.torch.cuda.synchronize()  # the sources stay alive until the copy ran

    def forward(self, kv, layer):
        self.blk.forward(self.x_d.data_ptr(), self.out.data_ptr(), self.b, self.s, self.mod_d.data_ptr(),
                         self.pe_d.data_ptr(), kv, layer, None, None, stream(self.torch))
        return host(self.out)

    def free(self):
        self.blk.free()


@pytest.fixture
def setup(torch_cuda, qctx):
    st = Setup(torch_cuda, qctx, 41)
    yield st
    st.free()


def test_host_cache_no_prefetch_matches_device(setup):
    kd, kh = setup.cache(False), setup.cache(True)
    for step in range(2):
        for layer in range(L):
            assert np.array_equal(setup.forward(kh, layer), setup.forward(kd, layer)), (step, layer)
    ref, _, _ = O.block_forward(SMALL, setup.w, setup.x, setup.mod, setup.pe, setup.k[2], setup.v[2], mode=O.CANDLE)
    got = setup.forward(kh, 2)
    assert cos_sim(got, ref) >= 0.9999 and max_abs_rel(got, ref) <= 2e-2
    kd.free()
    kh.free()


def test_host_cache_prefetch_on_copy_stream(setup):
    torch = setup.torch
    kd, kh = setup.cache(False), setup.cache(True)
    want = [setup.forward(kd, layer) for layer in range(L)]
    cs = torch.cuda.Stream()
    for step in range(3):
        kh.prefetch(0, cs.cuda_stream)
        for layer in range(L):
            if layer + 1 < L:
                kh.prefetch(layer + 1, cs.cuda_stream)
            assert np.array_equal(setup.forward(kh, layer), want[layer]), (step, layer)
    # irregular: prefetch ahead of use, twice, or not at all
    order = [("p", 3), ("p", 1), ("f", 2), ("f", 3), ("f", 1), ("p", 0), ("p", 0), ("f", 0), ("f", 3), ("p", 2),
             ("f", 1), ("f", 2)]
    for op, layer in order:
        if op == "p":
            kh.prefetch(layer, cs.cuda_stream)
        else:
            assert np.array_equal(setup.forward(kh, layer), want[layer]), (op, layer)
    torch.cuda.synchronize()
    kd.free()
    kh.free()


def test_host_cache_load_and_restore(setup):
    torch = setup.torch
    kh = setup.cache(True)
    shape = (setup.b, SMALL["heads"], setup.p, 128)
    for layer in range(L):
        k_o = torch.empty(shape, dtype=torch.int16, device="cuda")
        v_o = torch.empty_like(k_o)
        kh.load(layer, k_o.data_ptr(), v_o.data_ptr(), stream(torch))
        assert np.array_equal(host(k_o), setup.k[layer].view(np.int16))
        assert np.array_equal(host(v_o), setup.v[layer].view(np.int16))
    # stage layer 1, then store new contents into it: the forward sees the new ones
    cs = torch.cuda.Stream()
    kh.prefetch(1, cs.cuda_stream)
    setup.store(kh, 1, setup.k[3], setup.v[3])
    kd = setup.cache(False)
    assert np.array_equal(setup.forward(kh, 1), setup.forward(kd, 3))
    torch.cuda.synchronize()
    kd.free()
    kh.free()


def test_host_cache_rejects_bad_calls(setup):
    kh = setup.cache(True)
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        kh.prefetch(L, 0)
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        setup.qctx.kv_create_host(L, 1, 2, 8, head_dim=64)
    kh.free()
