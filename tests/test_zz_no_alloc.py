"""qimm_qmatmul_noalloc against qimm_qmatmul, through the C ABI: the same
kernels with the static per-device scratch in place of the context's growable
one, so the outputs must be bit-identical. Each case runs two calls in a row,
the second with fewer tokens, and interleaves calls of the allocating entry
point; the paths that use the scratch are all covered: the one-launch short-M
kernel (arrival counters + partial sums), the split 128x128 kernel (partials
+ the ordered reduction) and a large-M product whose last tile row goes to
the split path; the short-M kernels that keep their K sums inside a workgroup
run there too (no scratch)."""
import numpy as np
import pytest

import oracle as O
import synth
from gpu_util import bf16_dev, cos_sim, host, max_abs_rel, stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("t,m,m2,n,k,out", [
    (synth.Q4_K, 64, 16, 24576, 4096, synth.BF16),   # gate_up at 64 then 16 tokens: whole K per workgroup,
                                                     # then the in-workgroup K reduction (no partials)
    (synth.Q8_0, 64, 33, 12288, 4096, synth.BF16),   # q/k/v shape: one launch, split-K partials and counters
    (synth.Q6_K, 40, 5, 4096, 12288, synth.F32),     # down: twelve k chunks
    (synth.Q8_0, 256, 130, 4096, 4096, synth.BF16),  # split 128x128 (8 and 4 shares)
    (synth.Q4_K, 4352, 4136, 4096, 4096, synth.F32),  # large M: tail rows to the split / short-M paths
])
def test_qmatmul_noalloc_matches_qmatmul(torch_cuda, qctx, t, m, m2, n, k, out):
    torch = torch_cuda
    print(f"case: noalloc type {t} {n}x{k} at {m} then {m2} tokens", flush=True)
    rng = np.random.default_rng(m + n + k + t)
    _, w, _, _ = synth.weight(rng, t, n, k)
    W = qctx.upload(t, n, k, w.tobytes())
    a_dev, a = bf16_dev(torch, rng.standard_normal((m, k), dtype=np.float32))
    dt = torch.float32 if out == synth.F32 else torch.bfloat16
    for rows in (m, m2):
        y0 = torch.empty((rows, n), dtype=dt, device="cuda")
        y1 = torch.empty_like(y0)
        y2 = torch.empty_like(y0)
        qctx.qmatmul_noalloc(W, a_dev.data_ptr(), rows, k, y1.data_ptr(), out, stream(torch))
        qctx.qmatmul(W, a_dev.data_ptr(), rows, k, y0.data_ptr(), out, stream(torch))
        qctx.qmatmul_noalloc(W, a_dev.data_ptr(), rows, k, y2.data_ptr(), out, stream(torch))
        ref, g1, g2 = host(y0.float()), host(y1.float()), host(y2.float())
        assert np.array_equal(g1, ref) and np.array_equal(g2, ref), rows
        sel = np.unique(np.concatenate([np.arange(4), rng.choice(rows, min(8, rows), replace=False), np.arange(rows - 4, rows)]))
        want = O.qmatmul(t, w, n, k, a[sel], O.EXACT)
        assert cos_sim(g1[sel], want) >= 0.9999 and max_abs_rel(g1[sel], want) <= 2e-2
    W.free()


BLOCK_SHAPES = {"qkv": (12288, 4096), "out": (4096, 4096), "gate_up": (24576, 4096), "down": (4096, 12288)}


def test_scratch_bytes_of_the_block_projections_fit(torch_cuda, qctx):
    """qimm_qmatmul_scratch_bytes over every projection of the reference's block
    (hidden 4096, mlp 12288) in each weight format, at token counts across every
    kernel path: all within the static array of qimm_qmatmul_noalloc. A larger
    product (a bf16 weight of 204,800 rows at 64 tokens: one share of split-K
    partial sums, 64 x 204800 x 4 bytes) needs more, and the allocation-free
    entry point rejects it with QIMM_ERR_SHAPE."""
    import qimm
    limit = qimm_noalloc_bytes()
    rng = np.random.default_rng(9)
    worst = 0
    for t in (synth.Q8_0, synth.Q4_K, synth.Q6_K, synth.BF16):
        for name, (n, k) in BLOCK_SHAPES.items():
            W = qctx.upload(t, n, k, synth.random_blocks(rng, t, n, k).tobytes())
            for m in (1, 8, 16, 17, 33, 64, 65, 128, 256, 300, 511, 512, 1024, 2048, 4096, 4136, 4352, 8192):
                need = qctx.qmatmul_scratch_bytes(W, m)
                assert 0 <= need <= limit, (t, name, m, need)
                worst = max(worst, need)
            W.free()
    print(f"largest need over the block's projections: {worst / 2**20:.1f} MiB of {limit / 2**20:.0f}", flush=True)
    n, k = 204800, 256
    W = qctx.upload(synth.BF16, n, k, synth.random_blocks(rng, synth.BF16, n, k).tobytes())
    need = qctx.qmatmul_scratch_bytes(W, 64)
    print(f"bf16 {n}x{k} at 64 tokens needs {need / 2**20:.1f} MiB", flush=True)
    assert need > limit
    x = torch_cuda.zeros((64, k), dtype=torch_cuda.bfloat16, device="cuda")
    y = torch_cuda.empty((64, n), dtype=torch_cuda.bfloat16, device="cuda")
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        qctx.qmatmul_noalloc(W, x.data_ptr(), 64, k, y.data_ptr(), synth.BF16, stream(torch_cuda))
    W.free()


def qimm_noalloc_bytes():
    return 48 << 20  # QIMM_NOALLOC_SCRATCH_BYTES of include/qimm.h


def test_noalloc_product_and_reserved_block_under_graph_capture(torch_cuda, qctx):
    """The allocation-free product and a block forward after qimm_block_reserve,
    captured together in one torch.cuda graph (a capture stream of torch's): an
    allocation or a device-wide synchronize inside either call would fail the
    capture. The graph is replayed three times, with eager work of this
    program (buffer fills, the allocating product) and synchronizations
    between the replays, and every replay equals the eager results bit for bit."""
    import qimm
    from test_gpu_block import SMALL, block_tensors, make_case
    torch = torch_cuda
    print("case: graph capture of qmatmul_noalloc (Q8_0 12288x4096, 64 tokens) and a reserved block forward",
          flush=True)
    rng = np.random.default_rng(21)
    n, k, m = 12288, 4096, 64
    _, wq, _, _ = synth.weight(rng, synth.Q8_0, n, k)
    W = qctx.upload(synth.Q8_0, n, k, wq.tobytes())
    a_dev, _ = bf16_dev(torch, rng.standard_normal((m, k), dtype=np.float32))
    y_eager = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    y_graph = torch.empty_like(y_eager)
    w, x, mod, pe, kpre, vpre = make_case(22, SMALL, 1, 64, 16, synth.Q4_K, synth.Q6_K)
    keep = []
    blk = qctx.block_create(qimm.BlockConfig(SMALL["hidden"], SMALL["heads"], 128, SMALL["mlp"]),
                            block_tensors(w, keep))
    blk.reserve(1, 64)
    kv = qctx.kv_create(1, 1, SMALL["heads"], 16)
    kd = torch.from_numpy(kpre.view(np.int16)).cuda()
    vd = torch.from_numpy(vpre.view(np.int16)).cuda()
    kv.store(0, kd.data_ptr(), vd.data_ptr(), stream(torch))
    xd, md, ped = (torch.from_numpy(np.ascontiguousarray(v)).cuda() for v in (x, mod, pe))
    xo_eager, xo_graph = torch.empty_like(xd), torch.empty_like(xd)

    def calls(y, xo, sh):
        qctx.qmatmul_noalloc(W, a_dev.data_ptr(), m, k, y.data_ptr(), synth.BF16, sh)
        blk.forward(xd.data_ptr(), xo.data_ptr(), 1, 64, md.data_ptr(), ped.data_ptr(), kv, 0, None, None, sh)

    y_other = torch.empty_like(y_eager)
    # the allocating product runs between the replays: its scratch growth (a
    # free and an allocation of the context's split-K scratch, which the
    # captured block forward also uses) happens here, before the capture
    qctx.qmatmul(W, a_dev.data_ptr(), m, k, y_other.data_ptr(), synth.BF16, stream(torch))
    calls(y_eager, xo_eager, stream(torch))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        calls(y_graph, xo_graph, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        y_graph.fill_(0)
        xo_graph.fill_(0)
        qctx.qmatmul(W, a_dev.data_ptr(), m, k, y_other.data_ptr(), synth.BF16, stream(torch))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), rep
        assert torch.equal(xo_graph, xo_eager), rep
        assert torch.equal(y_other, y_eager), rep
    del g
    kv.free()
    blk.free()
    W.free()
