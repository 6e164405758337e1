"""Long shapes on paths the short parity cases do not reach.

* Five-slot key-tile ring: key tiles above 8 KiB (D=128: the screen stages
  fp16 K^ for every input type) stage through 5 LDS slots instead of 6.  At
  T=4096 a screen item walks up to 40 steps, so the ring wraps many times
  inside the straight-line loop.
* Cross-attention with a long key side (Tq=64, Tk=70000, non-causal, window
  wider than Tk): each bitmap row holds 2188 key units, more than one 2048-unit
  row load, in the live pass and in dQ.

Every output against the live-pair float64 oracle, max|got-ref|/max|ref| <=
1e-5 (fp32) or 2e-2 (bf16).
"""

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, np64, rel_err, head_sum_err, rw64

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
DEV = "cuda"


def _check(B, Tq, Tk, H, D, dtype, causal, r, w, seed):
    from multiscreen import ops
    print(f"long: B={B} Tq={Tq} Tk={Tk} H={H} D={D} {dtype} causal={causal} w={w}", flush=True)
    q, k, v = correlated_qkv(B, Tq, Tk, H, D, seed=seed, dtype=dtype, rho=0.35)
    dy = torch.randn(B, Tq, H, D, generator=torch.Generator().manual_seed(seed + 1)).to(dtype)
    rg, wg = torch.tensor(r, device=DEV), torch.tensor(w, device=DEV)
    qd, kd, vd, dyd = (t.to(DEV) for t in (q, k, v, dy))
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None)
    dq, dk, dv, dr, dw = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dyd)
    torch.cuda.synchronize()
    got = [np64(t) for t in (y, dq, dk, dv, dr, dw)]
    yref, gref, P = O.sparse_forward_backward(np64(q), np64(k), np64(v), rw64(r), rw64(w),
                                              np64(dy), causal)
    print(f"long: {len(P['i'])} live pairs", flush=True)
    tol = TOL[dtype]
    for name, g_, want in zip(("y", "dq", "dk", "dv", "dr", "dw"), got, (yref,) + tuple(gref)):
        assert np.max(np.abs(want)) > 0, f"{name} vacuous"
        e = rel_err(g_, want)
        assert e <= tol, f"{name}: rel err {e:.3e} > {tol}"
    # dr, dw entry by entry, against the sum of each head's |terms|
    for name, g_, want, scale in (("dr", got[4], gref[3], P["dr_abs"]), ("dw", got[5], gref[4], P["dw_abs"])):
        e = head_sum_err(g_, want, scale)
        assert e <= tol, f"{name}: per-head error {e:.3e} > {tol}"
    return P


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 128)], ids=["bf16_D128", "f32_D128"])
def test_five_slot_ring_long_items(dtype, D):
    _check(1, 4096, 4096, 2, D, dtype, True, [1.2, 1.35], [3000.0, 700.0], seed=31)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_cross_attention_long_key_rows(dtype):
    P = _check(1, 64, 70000, 1, 64, dtype, False, [1.3], [1e6], seed=41)
    # live keys past the first 2048 key units (65536 keys) of the rows
    assert np.any(P["j"] >= 65536)
