"""The C ABI of libmsa.so on the CPU: it loads, exports every function that
include/msa.h declares, and rejects bad arguments on the host before any HIP
call (so these run without a GPU)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT
from multiscreen import _native

HEADER = os.path.join(ROOT, "include", "msa.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(msa_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_header():
    L = _native.lib()
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), f"{n} declared in msa.h but not exported"
    # the ctypes binding covers exactly the declared set
    assert sorted(_native.EXPORTED) == names


def test_version_and_sizes():
    L = _native.lib()
    assert L.msa_version() == (0 << 16) | (3 << 8)
    # B=4, T=8192, H=8, D=64 bf16: one normalised K^ copy, then the screen's
    # work-plan table: 32 lanes x kmax entries of 32 bytes.  The size serves a
    # causal or a non-causal call: kmax = 68 causal (4 heads per XCD x 68
    # items of at most 40 steps, over 4 lanes), 128 non-causal (every group's
    # offsets span 131 tiles: 4 items a group), so 128
    one = 4 * 8 * 8192 * 64 * 2
    assert L.msa_fwd_workspace_bytes(4, 8, 8192, 8192, 64, 1) == one + 32 * 128 * 32
    # 2*nqt query-unit rows of ceil(2*nkt/32) words per (b, h)
    assert L.msa_tile_bits_words(4, 8, 8192, 8192) == 4 * 8 * 256 * 8
    assert L.msa_tile_bits_words(1, 1, 65, 65) == 4
    assert L.msa_tile_bits_words(1, 1, 64, 1100) == 2 * 2
    # D=16 is padded to 32 in the workspace; one head, one item per lane at
    # most; K^ is fp16 for every input type (fp32 inputs screen on fp16 too)
    assert L.msa_fwd_workspace_bytes(1, 1, 64, 64, 16, 0) == 64 * 32 * 2 + 1024
    # fp16 takes bf16's sizes (2-byte elements)
    assert L.msa_fwd_workspace_bytes(4, 8, 8192, 8192, 64, 2) == one + 32 * 128 * 32
    # backward workspace: (dr, dw) partial per (b, h, 32-query unit), then dh
    # (b, h, Tq_pad, DP) in the input type and 1/|q| (b, h, Tq_pad) fp32, each
    # 256-byte aligned
    assert L.msa_bwd_workspace_bytes(4, 8, 8192, 8192, 64, 1) == \
        2 * 4 * 8 * 256 * 4 + 4 * 8 * 8192 * 64 * 2 + 4 * 8 * 8192 * 4
    assert L.msa_bwd_workspace_bytes(1, 1, 65, 10, 16, 0) == 256 + 128 * 32 * 4 + 512
    assert L.msa_fwd_workspace_bytes(1, 1, 64, 64, 48, 0) == 0       # invalid D
    assert L.msa_decode_workspace_bytes(16, 8, 64, 100000) == 16 * 8 * 49 * 64 * 4


def _fwd(L, **kw):
    a = dict(q=16, qs=(1024, 64, 8), k=16, ks=(1024, 64, 8), v=16, vs=(1024, 64, 8),
             B=1, H=8, Tq=16, Tk=16, D=8 * 8, dtype=1, r=16, w=16, kpm=None, causal=1, eps=1e-8,
             drop=0.0, seed=0, y=16, hnorm=16, bits=16, nbits=16, ws=16, wsb=1 << 30, stream=None)
    a["D"] = 64
    a.update(kw)
    return L.msa_fwd(a["q"], *a["qs"], a["k"], *a["ks"], a["v"], *a["vs"], a["B"], a["H"], a["Tq"],
                     a["Tk"], a["D"], a["dtype"], a["r"], a["w"], a["kpm"], a["causal"], a["eps"],
                     a["drop"], a["seed"], a["y"], a["hnorm"], a["bits"], a["nbits"], a["ws"], a["wsb"], a["stream"])


@pytest.mark.parametrize("kw,code,msg", [
    (dict(D=48), 1, "head_dim"),
    (dict(dtype=3), 1, "dtype"),
    (dict(q=None), 1, "q is null"),
    (dict(q=24), 1, "aligned"),
    (dict(qs=(1024, 60, 8)), 1, "strides"),
    (dict(r=None), 1, "r and w"),
    (dict(nbits=0), 2, "tile_bits"),
    (dict(wsb=100), 2, "workspace"),
    (dict(eps=0.0), 1, "eps"),
    (dict(drop=1.0), 1, "dropout_p"),
    (dict(drop=-0.1), 1, "dropout_p"),
    (dict(B=70000, H=1), 1, "B*H"),
    (dict(Tq=-1), 1, "negative"),
])
def test_fwd_rejects_bad_arguments(kw, code, msg):
    L = _native.lib()
    rc = _fwd(L, **kw)
    assert rc == code
    assert msg in L.msa_last_error().decode()


def test_fwd_empty_batch_is_a_no_op():
    L = _native.lib()
    assert _fwd(L, B=0) == 0
    assert _fwd(L, Tq=0) == 0
    assert L.msa_last_error() == b""


def test_bwd_and_decode_reject_bad_arguments():
    L = _native.lib()
    rc = L.msa_bwd(16, 8, 8, 8, 16, 8, 8, 8, 16, 8, 8, 8, 1, 1, 8, 8, 16, 1, 16, 16, None, 1, 1e-8, 0.0, 0,
                   16, 16, 16, 16, 2, 16, 16, 16, 16, 16, 16, 10, None)
    assert rc == 2 and "backward workspace" in L.msa_last_error().decode()
    rc = L.msa_bwd(16, 8, 8, 8, 16, 8, 8, 8, 16, 8, 8, 8, 1, 1, 8, 8, 16, 1, 16, 16, None, 1, 1e-8, 0.0, 0,
                   16, 16, 16, 16, 0, 16, 16, 16, 16, 16, 16, 1 << 20, None)
    assert rc == 2 and "tile_bits" in L.msa_last_error().decode()
    rc = L.msa_decode(16, 512, 64, 16, 512, 512, 64, 16, 512, 512, 64, 1, 8, 64, 1, 0, 100, 0, 16, 16,
                      1e-8, 16, 16, 1 << 30, None)
    assert rc == 1 and "cache_len" in L.msa_last_error().decode()
    rc = L.msa_decode(16, 512, 64, 16, 512, 512, 64, 16, 512, 512, 64, 1, 8, 64, 1, 101, 100, 0, 16, 16,
                      1e-8, 16, 16, 1 << 30, None)
    assert rc == 1 and "capacity" in L.msa_last_error().decode()
    rc = L.msa_decode(16, 512, 64, 16, 512, 512, 64, 16, 512, 512, 64, 1, 8, 64, 1, 10, 100, 0, 16, 16,
                      1e-8, 16, 16, 8, None)
    assert rc == 2 and "decode workspace" in L.msa_last_error().decode()


def test_timer_rejects_unknown_kernel():
    L = _native.lib()
    assert L.msa_timer_arm(99, 1) == 1
    assert L.msa_timer_arm(0, 0) == 0
