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
