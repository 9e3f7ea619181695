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


def test_noalloc_first_call_inside_graph_capture(gpu):
    """Collected first in this file, so in a fresh process the entry point's first call (which resolves the device
    array's address and the error record) happens while a graph is being captured. The graph is replayed with
    three positions written in place, eager work between the replays, and every replay equals the workspace entry
    point run eagerly on the same inputs."""
    from lokinfer_amd import _lib

    L = _lib.lib()
    L.lk_hip_attention_decode_workspace_bytes.restype = C.c_int64
    dev = torch.device("cuda", 0)
    heads, cap = 12, 1024
    d = 64 * heads
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(1, 3 * d, generator=g).to(dev)
    bias = (0.1 * torch.randn(3 * d, generator=g)).to(dev)
    kc0 = torch.randn(cap, d, generator=g).to(dev)
    vc0 = torch.randn(cap, d, generator=g).to(dev)
    kc, vc = kc0.clone(), vc0.clone()
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    out = torch.zeros(1, d, device=dev)
    vp = C.c_void_p
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = L.lk_hip_attention_decode_f32_noalloc(
                vp(qkv.data_ptr()), vp(kc.data_ptr()), vp(vc.data_ptr()), vp(pos.data_ptr()), vp(bias.data_ptr()),
                vp(out.data_ptr()), C.c_int64(cap), C.c_int(heads), C.c_int64(cap), C.c_int(1),
                vp(side.cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    for p in (700, 3, 1023):
        kc.copy_(kc0)
        vc.copy_(vc0)
        pos.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        got = (out.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy())
        # the workspace entry point, eagerly, on the same inputs
        kw, vw = kc0.clone(), vc0.clone()
        ow = torch.zeros(1, d, device=dev)
        nbytes = L.lk_hip_attention_decode_workspace_bytes(heads, C.c_int64(cap))
        ws = torch.empty(nbytes // 4, device=dev)
        rc = L.lk_hip_attention_decode_f32(vp(qkv.data_ptr()), vp(kw.data_ptr()), vp(vw.data_ptr()),
                                           vp(pos.data_ptr()), vp(bias.data_ptr()), vp(ow.data_ptr()),
                                           C.c_int64(cap), C.c_int(heads), C.c_int64(cap), C.c_int(1),
                                           vp(ws.data_ptr()), C.c_int64(nbytes),
                                           vp(torch.cuda.current_stream(dev).cuda_stream))
        assert rc == 0
        torch.cuda.synchronize()
        assert np.isfinite(got[0]).all()
        for a, b in zip(got, (ow.cpu().numpy(), kw.cpu().numpy(), vw.cpu().numpy())):
            assert np.array_equal(a, b), p


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
