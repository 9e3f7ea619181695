"""The allocation-free decode attention entry point (lk_hip_attention_decode_f32_noalloc, partials in the library's
fixed device array) against the workspace entry point it shares its kernels with (lk_hip_attention_decode_f32):
bit-identical outputs and cache rows on two calls in a row, the second smaller, and a clear rejection of a call
beyond the array."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _call_pair(L, heads, cap, pos, seed):
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(seed)
    d = 64 * heads
    qkv = torch.randn(1, 3 * d, generator=g).to(dev)
    bias = (0.1 * torch.randn(3 * d, generator=g)).to(dev)
    kc0 = torch.randn(cap, d, generator=g).to(dev)
    vc0 = torch.randn(cap, d, generator=g).to(dev)
    p = torch.tensor([pos], dtype=torch.int64, device=dev)
    stream = C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    vp = C.c_void_p

    def run(noalloc):
        kc, vc = kc0.clone(), vc0.clone()
        out = torch.full((1, d), float("nan"), device=dev)
        args = [vp(qkv.data_ptr()), vp(kc.data_ptr()), vp(vc.data_ptr()), vp(p.data_ptr()), vp(bias.data_ptr()),
                vp(out.data_ptr()), C.c_int64(cap), C.c_int(heads), C.c_int64(cap), C.c_int(1)]
        if noalloc:
            rc = L.lk_hip_attention_decode_f32_noalloc(*args, stream)
        else:
            nbytes = L.lk_hip_attention_decode_workspace_bytes(heads, C.c_int64(cap))
            ws = torch.empty(nbytes // 4, device=dev)
            rc = L.lk_hip_attention_decode_f32(*args, vp(ws.data_ptr()), C.c_int64(nbytes), stream)
        assert rc == 0
        torch.cuda.synchronize()
        return out.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy()

    want = run(False)
    got = run(True)
    assert np.isfinite(want[0]).all()
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


def test_noalloc_decode_attention_matches_workspace_entry_point(gpu):
    from lokinfer_amd import _lib

    L = _lib.lib()
    L.lk_hip_attention_decode_noalloc_max_floats.restype = C.c_int64
    L.lk_hip_attention_decode_workspace_bytes.restype = C.c_int64
    _call_pair(L, heads=12, cap=1024, pos=700, seed=1)
    _call_pair(L, heads=4, cap=256, pos=100, seed=2)  # smaller: the array keeps the first call's partials past it


def test_noalloc_decode_attention_rejects_oversized_calls(gpu):
    from lokinfer_amd import _lib

    L = _lib.lib()
    L.lk_hip_attention_decode_noalloc_max_floats.restype = C.c_int64
    cap_max = L.lk_hip_attention_decode_noalloc_max_floats() // (64 * 66) * 64  # one head: ceil(cap / 64) * 66 floats
    vp = C.c_void_p
    # the size check runs before any pointer is touched or kernel launched
    rc = L.lk_hip_attention_decode_f32_noalloc(vp(0), vp(0), vp(0), vp(0), vp(0), vp(0), C.c_int64(cap_max + 64),
                                               C.c_int(64), C.c_int64(0), C.c_int(1), vp(0))
    assert rc == 4
