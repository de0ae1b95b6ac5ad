"""Helpers for the GPU parity tests: device buffers through torch, metrics of
the reference's probes (src/bin/quant_vs_full_probe.rs:13-17,
src/bin/kv_cache_probe.rs:11-14)."""
import numpy as np


def cos_sim(a, b):
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


def max_abs_rel(a, b):
    """max|a - b| / max|b| (b = reference)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def dev(torch, arr):
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bf16_dev(torch, x_f32):
    """f32 numpy -> bf16 device tensor (round to nearest even), plus its f32 value."""
    t = torch.from_numpy(np.ascontiguousarray(x_f32, dtype=np.float32)).to(torch.bfloat16)
    return t.cuda(), t.float().numpy()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def check_block(got_c, got_b, cand, exact, x):
    """Block outputs on the same token rows [R, hidden] in the two activation
    modes, against the oracle (x: their inputs).
    - got_c (QIMM_ACT_CANDLE, the reference CPU path's int8 activation
      rounding) against the oracle's candle mode: cosine >= 0.9999 and
      max|a-b|/max|b| <= 2e-2 on the output, and its update x_out - x at least
      as close to candle's update as the bf16 mode's is (the int8 rounding is
      really reproduced);
    - got_b (QIMM_ACT_BF16) against the oracle's exact mode: cosine >= 0.9999
      on the output and on the update, max|a-b|/max|b| <= 2e-2, and at least as
      close to exact arithmetic as the candle path is."""
    c_cc, u_cc = cos_sim(got_c, cand), cos_sim(got_c - x, cand - x)
    u_bc = cos_sim(got_b - x, cand - x)
    c_be, u_be = cos_sim(got_b, exact), cos_sim(got_b - x, exact - x)
    c_ce, u_ce = cos_sim(cand, exact), cos_sim(cand - x, exact - x)
    m_cc, m_be = max_abs_rel(got_c, cand), max_abs_rel(got_b, exact)
    print(f"candle mode vs candle: cos {c_cc:.7f} update {u_cc:.7f} mar {m_cc:.2e} (bf16 mode vs candle: update "
          f"{u_bc:.7f}); bf16 mode vs exact: cos {c_be:.7f} update {u_be:.7f} mar {m_be:.2e}; candle vs exact: "
          f"cos {c_ce:.7f} update {u_ce:.7f}", flush=True)
    assert c_cc >= 0.9999 and m_cc <= 2e-2
    assert u_cc >= u_bc
    assert c_be >= 0.9999 and u_be >= 0.9999 and m_be <= 2e-2
    assert c_be >= c_ce and u_be >= u_ce


def kv_close(got, want):
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2, (cos_sim(got, want),
                                                                            max_abs_rel(got, want))
