"""The allocation-free probe entry ``saf3r_probe_scores_noalloc`` called through the C ABI, checked
bit-exact against ``saf3r_probe_scores`` (caller workspace) on two calls in a row, the second with a
smaller input, so a result cannot come from the static workspace's previous contents."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def mods(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return importlib.import_module(pkg.__name__ + ".ops"), importlib.import_module(pkg.__name__ + "._lib")


def _probe(lib, L, noalloc, qk32, slots, sample):
    """Both probe entries through ctypes on fp32 q / k rows qk32 [n, 2, N, 64]."""
    n, N = len(slots), qk32.shape[2]
    hs = torch.tensor(slots, dtype=torch.int32, device=DEV)
    qbar = torch.full((n, 64), float("nan"), device=DEV)
    scores = torch.full((n, N + 3), float("nan"), device=DEV)
    sp = ctypes.c_void_p(0 if sample is None else sample.data_ptr())
    ns = 0 if sample is None else sample.numel()
    args = (ctypes.c_void_p(qk32.data_ptr()), ctypes.c_void_p(qk32[:, 1].data_ptr()), qk32.stride(0), N,
            ctypes.c_void_p(hs.data_ptr()), n, sp, ns, 0.125)
    outs = (ctypes.c_void_p(qbar.data_ptr()), ctypes.c_void_p(scores.data_ptr()), scores.stride(0), L.stream_ptr())
    if noalloc:
        rc = lib.saf3r_probe_scores_noalloc(*args, *outs)
    else:
        partial = torch.empty(n, 256, 64, device=DEV)
        rc = lib.saf3r_probe_scores(*args, ctypes.c_void_p(partial.data_ptr()), *outs)
    L.check(rc)
    torch.cuda.synchronize()
    return qbar.cpu(), scores[:, :N].cpu()


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_probe_matches_workspace_entry(mods, pkg, order):
    ops, L = mods
    lib = L.load()
    cases = [(6 * 1374, [5, 0, 3, 7, 1, 2, 6, 4], None),                          # 8 heads, every token
             (2 * 155, [1, 2], torch.tensor([0, 7, 150, 309], dtype=torch.int32))]  # smaller, sampled rows
    for i, (N, slots, sample) in enumerate(cases):
        print(f"call {i}: N {N} slots {slots} sample {None if sample is None else sample.tolist()}", flush=True)
        g = torch.Generator().manual_seed(20 + i)
        qk32 = (torch.randn(max(slots) + 1, 2, N, 64, generator=g) * 2).to(DEV)
        s = None if sample is None else sample.to(DEV)
        want_q, want_s = _probe(lib, L, False, qk32, slots, s)
        got_q, got_s = _probe(lib, L, True, qk32, slots, s)
        assert np.array_equal(got_q.numpy().view(np.uint32), want_q.numpy().view(np.uint32)), f"qbar, call {i}"
        assert np.array_equal(got_s.numpy().view(np.uint32), want_s.numpy().view(np.uint32)), f"scores, call {i}"
        assert torch.isfinite(got_s).all()


def test_noalloc_probe_rejects_more_heads_than_the_workspace(mods, pkg):
    """65 heads exceed the static workspace's 64: rejected before any launch. Every buffer is a real
    device tensor of the size the call describes, so that a rejection that stopped working would show
    as a wrong status, not as an access to an invalid address."""
    ops, L = mods
    lib = L.load()
    n_sel, n_tok = 65, 64
    qk32 = torch.zeros(n_sel, 2, n_tok, 64, device=DEV)
    slots = torch.arange(n_sel, dtype=torch.int32, device=DEV)
    qbar = torch.zeros(n_sel, 64, device=DEV)
    scores = torch.zeros(n_sel, n_tok, device=DEV)
    torch.cuda.synchronize()
    rc = lib.saf3r_probe_scores_noalloc(ctypes.c_void_p(qk32.data_ptr()), ctypes.c_void_p(qk32[:, 1].data_ptr()),
                                        qk32.stride(0), n_tok, ctypes.c_void_p(slots.data_ptr()), n_sel, None, 0,
                                        0.125, ctypes.c_void_p(qbar.data_ptr()), ctypes.c_void_p(scores.data_ptr()),
                                        scores.stride(0), L.stream_ptr())
    torch.cuda.synchronize()
    assert rc == 2 and b"static workspace" in lib.saf3r_last_error()
    assert (qbar == 0).all() and (scores == 0).all()  # nothing was launched


def test_noalloc_probe_on_a_side_stream(mods, pkg):
    """On a non-default stream the entry resolves its workspace from the stream's device
    (hipStreamGetDevice): the same results as the workspace entry on that stream."""
    ops, L = mods
    lib = L.load()
    g = torch.Generator().manual_seed(31)
    N, slots = 3 * 155, [2, 0]
    qk32 = (torch.randn(3, 2, N, 64, generator=g) * 2).to(DEV)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        assert L.stream_ptr().value  # a real stream handle, not the NULL stream
        want_q, want_s = _probe(lib, L, False, qk32, slots, None)
        got_q, got_s = _probe(lib, L, True, qk32, slots, None)
    assert np.array_equal(got_q.numpy().view(np.uint32), want_q.numpy().view(np.uint32))
    assert np.array_equal(got_s.numpy().view(np.uint32), want_s.numpy().view(np.uint32))
