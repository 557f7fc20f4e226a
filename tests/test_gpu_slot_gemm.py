"""The decode step's GEMM (slot_gemm.hip, through dec_debug_slot_gemm) against torch in float64: every epilogue, ragged
row and slot counts, split-K slice counts; determinism; a slot's result independent of the other slots (alone, among
others, at another place); and the shapes it declines."""
import numpy as np
import pytest
import torch

from nanochat_amd.native import hip_library, pointer, stream

pytestmark = pytest.mark.gpu

STORE, RESID2, RELU2, RESID, F32 = range(5)
# the config-5 decode shapes (qkv, o, fc, proj, lm_head) at full and partial slot counts, and ragged small ones; across
# their slice counts they use every workgroup tile (tests/test_abi.py checks which)
SHAPES = [(4992, 1664, 128), (1664, 1664, 1), (6656, 1664, 37), (1664, 6656, 128), (100, 128, 16), (36, 256, 65),
          (65536, 1664, 100), (260, 384, 17)]


def bf16_ulp(x):
    """bf16 spacing at |x| (2^-133 floor for zeros)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def run(epi, w, x, res=None, rstd=None, slices=0):
    R, K = w.shape
    N = x.shape[0]
    dev = w.device
    out = torch.full((N, R), 7.0, dtype=torch.bfloat16, device=dev)
    out32 = torch.full((N, R), 7.0, dtype=torch.float32, device=dev)
    lib = hip_library("decode")
    S = slices or lib.dec_debug_slot_gemm_slices(R, K)
    part = torch.empty(max(1, lib.dec_debug_slot_gemm_part_bytes(R, N, S) // 4), dtype=torch.float32, device=dev)
    print(f"slot_gemm epi={epi} R={R} K={K} N={N} S={S}", flush=True)
    st = lib.dec_debug_slot_gemm(epi, pointer(w), R, K, pointer(x), N, pointer(out), pointer(out32),
                                 pointer(res) if res is not None else None,
                                 pointer(rstd) if rstd is not None else None, slices, pointer(part), stream())
    assert st == 0, st
    torch.cuda.synchronize()
    return out, out32


# every shape at its default slice count and at 1, 2 and 3 slices where it has that many 128-wide chunks
CASES = [(R, K, N, S) for R, K, N in SHAPES for S in (0, 1, 2, 3) if S <= K // 128]


@pytest.mark.parametrize("R,K,N,slices", CASES)
def test_epilogues_match_float64(device, R, K, N, slices):
    gen = torch.Generator().manual_seed(R * 7 + K + N)
    w = (torch.randn(R, K, generator=gen) * 0.05).bfloat16()
    x = torch.randn(N, K, generator=gen).bfloat16()
    res = torch.randn(N, R, generator=gen).bfloat16()
    rstd = torch.rand(N, generator=gen) + 0.5
    s = x.double() @ w.double().T                                  # exact products, float64 sums
    bound = (x.double().abs() @ w.double().abs().T) * K * 2.0 ** -24  # fp32 accumulation error bound
    wd, xd, rd, sd = w.to(device), x.to(device), res.to(device), rstd.to(device)

    out, f32 = run(F32, wd, xd, slices=slices)
    assert torch.all(out.cpu() == 7.0)                             # F32 writes only the fp32 output
    f32 = f32.cpu().double()
    assert (f32 - s).abs().le(bound + 1e-30).all()

    def check_bf16(out, ref, prop, label):
        """bf16(f(s_device)) against f(s): one bf16 rounding plus the propagated accumulation error `prop`."""
        got = out.cpu().double().numpy()
        ref, prop = ref.numpy(), prop.numpy()
        assert np.all(np.abs(got - ref) <= bf16_ulp(ref) + prop + 1e-30), label

    out, o32 = run(STORE, wd, xd, slices=slices)
    check_bf16(out, s, bound, "store")
    assert torch.all(o32.cpu() == 7.0)
    out, o32 = run(RESID2, wd, xd, res=rd, slices=slices)
    xsum = s + res.double()
    check_bf16(out, xsum, bound + 2.0 ** -24 * xsum.abs(), "resid2 bf16")
    assert (o32.cpu().double() - xsum).abs().le(bound + 2.0 ** -24 * xsum.abs() + 1e-30).all()
    out, _ = run(RELU2, wd, xd, rstd=sd, slices=slices)
    r = rstd.double()[:, None]
    p = s * r
    check_bf16(out, torch.relu(p) * p, 2 * p.abs() * r * bound + (r * bound) ** 2 + 2.0 ** -22 * p * p, "relu2")
    out, _ = run(RESID, wd, xd, res=rd, slices=slices)
    check_bf16(out, xsum, bound + 2.0 ** -24 * xsum.abs(), "resid")


def test_deterministic_and_declines_bad_shapes(device):
    gen = torch.Generator().manual_seed(5)
    w = (torch.randn(1664, 6656, generator=gen) * 0.05).bfloat16().to(device)
    x = torch.randn(128, 6656, generator=gen).bfloat16().to(device)
    a = run(F32, w, x)[1]
    b = run(F32, w, x)[1]
    assert torch.equal(a, b)
    lib = hip_library("decode")
    out = torch.empty(256, 1664, dtype=torch.float32, device=device)
    x2 = torch.zeros(129, 6656, dtype=torch.bfloat16, device=device)
    for R, K, N, xx in ((1664, 6656, 129, x2), (1664, 6600, 128, x), (1662, 6656, 128, x)):
        assert lib.dec_debug_slot_gemm(F32, pointer(w), R, K, pointer(xx), N, None, pointer(out), None, None, 1,
                                       None, stream()) == -2


@pytest.mark.parametrize("R,K", [(4992, 1664), (1664, 6656)])
def test_a_slots_result_does_not_depend_on_the_others(device, R, K):
    """Slot rows are summed in one fixed order whatever N is and whatever workgroup tile holds them: a row computed
    alone, among 128 others, at another place and among 37 gives the same bits (the decoder's batch independence rests
    on this; the three slot counts use different tiles)."""
    lib = hip_library("decode")
    assert len({lib.dec_debug_slot_gemm_tile(R, K, n, 0) for n in (1, 37, 128)}) >= 2
    gen = torch.Generator().manual_seed(R + K)
    w = (torch.randn(R, K, generator=gen) * 0.05).bfloat16().to(device)
    x = torch.randn(128, K, generator=gen).bfloat16().to(device)
    full = run(F32, w, x)[1]
    for n in (0, 5, 77, 127):
        alone = run(F32, w, x[n:n + 1].contiguous())[1]
        assert torch.equal(alone[0], full[n]), n
    order = torch.randperm(128, generator=torch.Generator().manual_seed(3)).to(device)
    moved = run(F32, w, x[order].contiguous())[1]
    assert torch.equal(moved, full[order])
    part = run(F32, w, x[40:77].contiguous())[1]
    assert torch.equal(part, full[40:77])


@pytest.mark.parametrize("R,K,N", [(1664, 1664, 128), (6656, 1664, 37), (260, 384, 17), (1664, 1664, 1)])
def test_mlp_rstd_from_tile_sums(device, R, K, N):
    """The step's MLP rstd without its own kernel: the o GEMM (RESID2) writes each 16-row tile's sum of squares of its
    residual sum x = s + res, and the fc GEMM (RELU2) takes rstd = 1 / sqrt(sum / K + FLT_EPSILON) from the tiles of
    its K = C row. Against float64: the tile sums (fp32 accumulation bound), then fc's output from an x whose rows are
    the o GEMM's (one GEMM run as both, R = K)."""
    lib = hip_library("decode")
    gen = torch.Generator().manual_seed(R + K + N)
    w = (torch.randn(R, K, generator=gen) * 0.05).bfloat16()
    x = torch.randn(N, K, generator=gen).bfloat16()
    res = torch.randn(N, R, generator=gen).bfloat16()
    tiles = -(-R // 16)
    s = x.double() @ w.double().T
    bound = (x.double().abs() @ w.double().abs().T) * K * 2.0 ** -24
    xs = s + res.double()
    out = torch.full((N, R), 7.0, dtype=torch.bfloat16, device=device)
    ssq = torch.full((N, tiles), -1.0, dtype=torch.float32, device=device)
    print(f"slot_gemm ssq RESID2 R={R} K={K} N={N}", flush=True)
    assert lib.dec_debug_slot_gemm_ssq(1, pointer(w.to(device)), R, K, pointer(x.to(device)), N, pointer(out),
                                       pointer(res.to(device)), pointer(ssq), stream()) == 0
    torch.cuda.synchronize()
    got = out.cpu().double().numpy()
    assert np.all(np.abs(got - xs.numpy()) <= bf16_ulp(xs.numpy()) + (bound + 2.0 ** -24 * xs.abs()).numpy() + 1e-30)
    pad = torch.zeros(N, tiles * 16, dtype=torch.float64)
    pad[:, :R] = xs
    want = (pad.view(N, tiles, 16) ** 2).sum(-1)
    err_x = bound + 2.0 ** -24 * xs.abs()                    # |x_device - x| per element
    pad_e = torch.zeros_like(pad)
    pad_e[:, :R] = err_x * (2 * xs.abs() + err_x)             # |x_d^2 - x^2|
    tol = pad_e.view(N, tiles, 16).sum(-1) + want * 32 * 2.0 ** -24
    assert ((ssq.cpu().double() - want).abs() <= tol).all()

    # fc: K = R of the o GEMM above, rstd from those tile sums
    if R != K:
        return
    w2 = (torch.randn(3 * K, K, generator=gen) * 0.05).bfloat16()
    x2 = out.cpu()                                           # the o GEMM's bf16 output as fc's input
    u = torch.full((N, 3 * K), 7.0, dtype=torch.bfloat16, device=device)
    print(f"slot_gemm ssq RELU2 R={3 * K} K={K} N={N}", flush=True)
    assert lib.dec_debug_slot_gemm_ssq(2, pointer(w2.to(device)), 3 * K, K, pointer(x2.to(device)), N, pointer(u),
                                       None, pointer(ssq), stream()) == 0
    torch.cuda.synchronize()
    ss = ssq.cpu().double().sum(-1)
    r = (1.0 / torch.sqrt(ss / K + 2.0 ** -23))[:, None]
    s2 = x2.double() @ w2.double().T
    b2 = (x2.double().abs() @ w2.double().abs().T) * K * 2.0 ** -24
    p = s2 * r
    ref = torch.relu(p) * p
    # the device's rstd differs from r by its fp32 sum over <= 128 tiles and one sqrt / divide
    rerr = r * (128 * 2.0 ** -24 + 2.0 ** -22)
    perr = b2 * r + s2.abs() * rerr
    tol2 = 2 * p.abs() * perr + perr ** 2 + 2.0 ** -22 * p * p
    assert np.all(np.abs(u.cpu().double().numpy() - ref.numpy()) <= bf16_ulp(ref.numpy()) + tol2.numpy() + 1e-30)
    assert lib.dec_debug_slot_gemm_ssq(2, pointer(w2.to(device)), 3 * K, K, pointer(x2.to(device)), N, pointer(u),
                                       None, None, stream()) == -2
