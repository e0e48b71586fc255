"""The kernel-level binding of the reference's Triton entry points (``kernel_binding``), through the
C ABI, against the CPU oracle: ``compute_qk_topk_indices_fused`` over a batch of two (both top-k
paths, the larger one through the caller-owned score workspace) and ``fused_sparse_topk_attention``
in the reference's output dtype (``v.dtype``) for bf16, fp16 and fp32 inputs.

Bars: top-k indices identical except within fp32 accumulation noise of a tie (the MFMA summation
order is not the oracle's), selected scores within 1e-4; gather outputs in bf16 within max-abs 2e-2 /
mean-abs 2e-3, with fp32 / fp16 values within 1e-4 / 2e-3 of the fp64 oracle (fp32 arithmetic
throughout, about 1e-5 of score error at these magnitudes; fp16 adds its one output rounding, half
an ulp of at most 1e-3 below 4)."""
import importlib

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selection as OS

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def kb(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return importlib.import_module(pkg.__name__ + ".kernel_binding")


def _check_topk(got, q, k, frames, topk):
    s = (q.double() @ k.double().T).float().numpy()  # exact products of the bf16 values, fp32 sums
    ref = OS.frame_topk(s, frames, topk)
    assert got.shape == ref.shape
    gs = np.take_along_axis(s, got.astype(np.int64), axis=1)
    rs = np.take_along_axis(s, ref.astype(np.int64), axis=1)
    assert np.allclose(gs, rs, atol=1e-4, rtol=0), "selected scores differ beyond rounding noise"
    assert (got == ref).mean() >= 0.99
    return ref


@pytest.mark.parametrize("topk", [4, 24])
def test_compute_qk_topk_indices_fused_batch_of_two(kb, topk):
    """B = 2 with different q and k per batch element: each element against its own oracle, and
    element 1 against a call of its own (no batch is dropped or mixed up)."""
    B, nq, frames, P = 2, 333, 3, 150
    g = torch.Generator().manual_seed(40 + topk)
    q = torch.randn(B, nq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(B, frames * P, 64, generator=g).to(torch.bfloat16)
    got = kb.compute_qk_topk_indices_fused(q.to(DEV), k.to(DEV), topk, P)
    torch.cuda.synchronize()
    assert got.shape == (B, nq, frames * min(topk, P)) and got.dtype == torch.int32
    got = got.cpu().numpy()
    for b in range(B):
        print(f"batch {b} topk {topk}", flush=True)
        _check_topk(got[b], q[b], k[b], frames, topk)
    alone = kb.compute_qk_topk_indices_fused(q[1:].to(DEV), k[1:].to(DEV), topk, P).cpu().numpy()
    assert np.array_equal(alone[0], got[1])
    assert not np.array_equal(got[0], got[1])


def test_compute_qk_topk_indices_fused_fp32_inputs_round_to_bf16(kb):
    """fp32 q / k are rounded to bf16 first, as the reference's kernel multiplies bf16 tiles."""
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 200, 64, generator=g)
    k = torch.randn(1, 2 * 90, 64, generator=g)
    got = kb.compute_qk_topk_indices_fused(q.to(DEV), k.to(DEV), 5, 90)
    want = kb.compute_qk_topk_indices_fused(q.to(torch.bfloat16).to(DEV), k.to(torch.bfloat16).to(DEV), 5, 90)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want.cpu())


def test_binding_rejects_unsupported_sizes(kb):
    q = torch.randn(10, 32, device=DEV)
    with pytest.raises(ValueError, match="D = Dv = 64"):
        kb.fused_sparse_topk_attention(q, q, q, torch.zeros(10, 3, dtype=torch.int32, device=DEV))
    q64 = torch.randn(10, 64, device=DEV)
    with pytest.raises(ValueError, match="D = Dv = 64"):
        kb.fused_sparse_topk_attention(q64, q64, torch.randn(10, 128, device=DEV),
                                       torch.zeros(10, 3, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError, match="D = 64"):
        kb.compute_qk_topk_indices_fused(torch.randn(1, 10, 32, device=DEV), torch.randn(1, 20, 32, device=DEV),
                                         4, 10)
    with pytest.raises(ValueError, match="divisible"):
        kb.compute_qk_topk_indices_fused(torch.randn(1, 10, 64, device=DEV), torch.randn(1, 25, 64, device=DEV),
                                         4, 10)
    with pytest.raises(ValueError, match="1 .. 128"):
        kb.compute_qk_topk_indices_fused(torch.randn(1, 10, 64, device=DEV), torch.randn(1, 400, 64, device=DEV),
                                         129, 200)


@pytest.mark.parametrize("vdt,qkdt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                      (torch.float32, torch.float32), (torch.float16, torch.float16),
                                      (torch.float32, torch.bfloat16)])
def test_fused_sparse_topk_attention_dtypes(kb, vdt, qkdt):
    """out in v.dtype from fp32 arithmetic on the upcast inputs; -1 entries skipped; a stride-0 list."""
    n, nk, topk = 150, 700, 96
    g = torch.Generator().manual_seed(3)
    q, k = ((2.0 * torch.randn(m, 64, generator=g)).to(qkdt) for m in (n, nk))
    v = torch.randn(nk, 64, generator=g).to(vdt)
    idx = torch.randint(0, nk, (n, topk), generator=g, dtype=torch.int32)
    idx[0, :5] = -1
    got = kb.fused_sparse_topk_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV))
    shared = kb.fused_sparse_topk_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx[3:4].expand(n, topk).to(DEV))
    torch.cuda.synchronize()
    assert got.dtype == vdt and got.shape == (n, 64)
    for out, lst in ((got, idx), (shared, idx[3:4].expand(n, topk).contiguous())):
        ref = OA.gather_attention(q.double(), k.double(), v.double(), lst, dtype=torch.float64)
        err = (out.cpu().double() - ref).abs()
        print(f"v {vdt} qk {qkdt}: max {err.max().item():.3g} mean {err.mean().item():.3g}", flush=True)
        if vdt == torch.float32:
            assert err.max().item() <= 1e-4
        elif vdt == torch.float16:
            assert err.max().item() <= 2e-3
        else:
            assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
