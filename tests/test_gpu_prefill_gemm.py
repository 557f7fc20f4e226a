"""The decoder's prefill GEMM (prefill_gemm.hip, through dec_debug_prefill_gemm) against float64 products on the CPU,
at config 5's shapes (qkv 4,992 x 1,664, o 1,664 x 1,664, fc 6,656 x 1,664, proj 1,664 x 6,656) and a small model's, with
row counts that leave partial tiles in both dimensions. Each epilogue: fp32 sums within fp32 accumulation error of the
float64 product; bf16(s), bf16(s + res) and bf16(relu(p) p), p = s rstd, within one bf16 rounding of the same made from
the float64 sum. And batch independence: a row's bits are the same whatever M holds (rows 0..36 alone, in 300 rows and
in 8,192 rows), as dec_prefill needs for a prompt to give the same cache in any call."""
import numpy as np
import pytest
import torch

from nanochat_amd.native import hip_library, pointer, stream

pytestmark = pytest.mark.gpu

STORE, RELU2, RESID, F32 = 0, 2, 3, 4


def run(epi, w, a, res=None, rstd=None):
    M, K = a.shape
    N = w.shape[0]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    out_f32 = torch.empty(M, N, dtype=torch.float32, device=a.device)
    rc = hip_library("decode").dec_debug_prefill_gemm(
        epi, pointer(w), N, K, pointer(a), M, pointer(out), pointer(out_f32),
        pointer(res) if res is not None else None, pointer(rstd) if rstd is not None else None, stream())
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out_f32 if epi == F32 else out


def bf16_np(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().float().numpy().astype(np.float64)


@pytest.mark.parametrize("N,K,M", [(4992, 1664, 300), (1664, 1664, 530), (6656, 1664, 257), (1664, 6656, 130),
                                   (768, 256, 77), (1024, 256, 1)])
def test_prefill_gemm_matches_float64(device, N, K, M):
    gen = torch.Generator().manual_seed(N + K + M)
    w = (torch.randn(N, K, generator=gen) * 0.02).bfloat16()
    a = torch.randn(M, K, generator=gen).bfloat16()
    res = torch.randn(M, N, generator=gen).bfloat16()
    rstd = (0.5 + torch.rand(M, generator=gen)).float()
    ref = a.double().numpy() @ w.double().numpy().T                     # exact products, float64 sums
    wd, ad = w.to(device), a.to(device)
    s32 = run(F32, wd, ad).double().cpu().numpy()
    # fp32 accumulation over K terms: within K * 2^-24 of the sum of |products|
    bound = K * 2.0 ** -24 * (np.abs(a.double().numpy()) @ np.abs(w.double().numpy()).T) + 1e-30
    assert (np.abs(s32 - ref) <= bound).all()
    for epi in (STORE, RESID, RELU2):
        got = run(epi, wd, ad, res.to(device), rstd.to(device)).double().cpu().numpy()
        if epi == STORE:
            want = ref
        elif epi == RESID:
            want = ref + res.double().numpy()
        else:
            p = ref * rstd.double().numpy()[:, None]
            want = np.maximum(p, 0.0) * p
        # one bf16 rounding (2^-8 relative) plus the fp32 sum's error carried through
        tol = 2.0 ** -8 * np.abs(want) + 4 * bound * (1 + (np.abs(ref) * rstd.double().numpy()[:, None] if epi == RELU2
                                                           else 0)) + 1e-6
        assert (np.abs(got - want) <= tol).all(), (epi, float(np.abs(got - want).max()))


def test_prefill_gemm_rows_do_not_depend_on_m(device):
    gen = torch.Generator().manual_seed(9)
    N, K = 4992, 1664
    w = (torch.randn(N, K, generator=gen) * 0.02).bfloat16().to(device)
    a = torch.randn(8192, K, generator=gen).bfloat16().to(device)
    full = run(STORE, w, a)
    mid = run(STORE, w, a[:300].contiguous())
    small = run(STORE, w, a[:37].contiguous())
    assert torch.equal(full[:300].view(torch.int16), mid.view(torch.int16))
    assert torch.equal(full[:37].view(torch.int16), small.view(torch.int16))
    # and a row in a later tile, moved to row 0 of a call of its own
    one = run(STORE, w, a[5000:5001].contiguous())
    assert torch.equal(full[5000:5001].view(torch.int16), one.view(torch.int16))


@pytest.mark.parametrize("N,K,M,epi", [(4992, 1664, 8192, STORE), (6656, 1664, 8192, RELU2), (6656, 1664, 5000, F32)])
def test_split_tiles_match_whole_tiles(device, N, K, M, epi):
    """At these sizes the last round's tiles are cut into halves (qkv: 640 tiles, 128 of them in halves) or quarters
    (fc: 832 tiles, 64 in quarters; 5,000 rows: 520 tiles, 8 in quarters, some past M); every output must equal the
    same row computed in 256-row calls, whose few tiles are never cut."""
    gen = torch.Generator().manual_seed(N + M + epi)
    w = (torch.randn(N, K, generator=gen) * 0.02).bfloat16().to(device)
    a = torch.randn(M, K, generator=gen).bfloat16().to(device)
    rstd = (0.5 + torch.rand(M, generator=gen)).float().to(device)
    full = run(epi, w, a, rstd=rstd)
    bits = torch.int32 if epi == F32 else torch.int16
    for r0 in range(0, M, 256):
        r1 = min(M, r0 + 256)
        part = run(epi, w, a[r0:r1].contiguous(), rstd=rstd[r0:r1].contiguous())
        assert torch.equal(full[r0:r1].view(bits), part.view(bits)), (r0, r1)
