"""msa_decode_noalloc: the decode entry point that allocates nothing (its
partial sums live in a static device array).  Checked through the C ABI
against msa_decode with a caller workspace -- the same kernels, so the
outputs must be bitwise equal -- on two calls in a row, both taking the
split launch that writes and reads the static array, the second with fewer
heads and a shorter cache (it reads back partials over the ones the first
call left), and against the oracle's decode row; oversize calls are rejected before any
device work."""

import math

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, np64, rel_err, rw64

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _lib():
    from multiscreen import _native
    return _native.lib()


def _decode(L, q, kc, vc, n, r, w, hint, static):
    B, H, D = q.shape
    dt = 1 if q.dtype == torch.bfloat16 else 0
    y = torch.empty_like(q)
    args = (q.data_ptr(), q.stride(0), q.stride(1),
            kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
            vc.data_ptr(), vc.stride(0), vc.stride(1), vc.stride(2),
            B, H, D, dt, n, kc.shape[1], hint, r.data_ptr(), w.data_ptr(), 1e-8, y.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    if static:
        rc = L.msa_decode_noalloc(*args, stream)
    else:
        nbytes = int(L.msa_decode_workspace_bytes(B, H, D, n))
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
        rc = L.msa_decode(*args, ws.data_ptr(), nbytes, stream)
    assert rc == 0, L.msa_last_error().decode()
    return y


@pytest.mark.gpu
def test_decode_noalloc_matches_decode_on_consecutive_calls():
    L = _lib()
    cases = [
        # B, T, H, D, dtype, cache_len, hint, r, w
        (4, 6000, 8, 64, torch.bfloat16, 6000, 0, [1.1, 1.2, 1.3, 1.5, 2.0, 1.15, 1.25, 1.1],
         [3.0, 40.0, 300.0, 2100.0, 5000.0, 1e5, 7.5, 4097.0]),
        # second call: fewer heads and a shorter cache, still over one 2048-key
        # chunk with hint 0, so it takes the split launch and its partials go
        # to the static array the first, larger call has left full
        (2, 5000, 3, 32, torch.float32, 4500, 0, [1.1, 1.2, 1.4], [2.0, 3000.0, 1e6]),
    ]
    L_chunk = 2048
    assert all(n > L_chunk and hint == 0 for _, _, _, _, _, n, hint, _, _ in cases)
    assert cases[1][0] * cases[1][2] < cases[0][0] * cases[0][2]
    for B, T, H, D, dtype, n, hint, r, w in cases:
        q, k, v = correlated_qkv(B, T, T, H, D, seed=21, dtype=dtype, rho=0.35)
        qd = q[:, n - 1].to("cuda").contiguous()
        kc, vc = k.to("cuda"), v.to("cuda")
        rg = torch.tensor(r, dtype=torch.float32, device="cuda")
        wg = torch.tensor(w, dtype=torch.float32, device="cuda")
        want = _decode(L, qd, kc, vc, n, rg, wg, hint, static=False)
        got = _decode(L, qd, kc, vc, n, rg, wg, hint, static=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (B, T, H, D, n)
        ref = O.decode_row(np64(q[:, n - 1]), np64(k), np64(v), n, rw64(r), rw64(w))
        assert np.max(np.abs(ref)) > 1e-3
        assert rel_err(np64(got), ref, heads=(0, 1)) <= TOL[dtype]


def test_decode_noalloc_rejects_sizes_beyond_its_scratch():
    # 16 * 8 heads * 2048 chunks * 64 floats = 64 MiB of partials > 16 MiB:
    # rejected on the host before any device work (no GPU needed)
    L = _lib()
    rc = L.msa_decode_noalloc(16, 512, 64, 16, 512, 512, 64, 16, 512, 512, 64, 16, 8, 64, 1, 1 << 22, 1 << 22, 0,
                              16, 16, 1e-8, 16, None)
    assert rc == 2
    msg = L.msa_last_error().decode()
    assert "static scratch" in msg and str(16 << 20) in msg
