"""Kernel-level parity of the HIP path (through the C ABI) against plain fp32 references of the same op, at the
vision / decoder / TRecViT shapes (the reference's kernel regression test, moondream/gpu/test_hgemm.py:15-50, with
asserting tolerances). References are computed in fp32 on the CPU."""
import pytest
import torch
import torch.nn.functional as F

import strix_halo_maxx_amd.ops as ops
from strix_halo_maxx_amd import _lib

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def within_ulps(a, b, n=1, frac=1e-3):
    """|a - b| <= n bf16 ulps everywhere, and a != b on at most `frac` of the elements."""
    a, b = a.float().cpu(), b.float().cpu()
    tol = n * 2.0 ** -7 * torch.maximum(a.abs(), b.abs()) + 1e-30
    return bool(((a - b).abs() <= tol).all()) and (a != b).float().mean().item() <= frac


def gen(seed):
    return torch.Generator().manual_seed(seed)


GEMM_SHAPES = [(729, 1152, 3456), (729, 1152, 1152), (729, 1152, 4304), (729, 4304, 1152), (729, 592, 1152),
               (1, 2048, 6144), (37, 2048, 2048), (1280, 768, 1536), (1458, 1152, 1152)]


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
def test_gemm_bias_vs_fp32(dev, M, K, N):
    g = gen(M * 7 + N)
    x = torch.randn(M, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    ref = x.float() @ w.float().t() + b.float()
    lin = ops.MxLin(w, b)
    print(f"gemm M={M} K={K} N={N}", flush=True)
    y = lin(x.to(dev))
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == BF
    assert rel(y, ref) < 5e-3
    # the output is the bf16 rounding of an fp32 accumulation: within 1 bf16 ulp-ish of the fp32 result
    assert (y.float().cpu() - ref).abs().max().item() < 0.02 * ref.abs().max().item() + 1e-2


NCFG = 28  # tile configs the library exports
# 8-wave tiles, the 4-wave 256 x 256 tile and the 192 x 192 two-k-group tile: no partial-sum mode, no split-K
NO_PSUM = {15, 16, 17, 18, 24, 25}
KH2 = {19, 20, 21, 22, 26, 27}  # 2 x 2 tiles over two k groups of waves: partial-sum mode, no in-kernel split-K


@pytest.mark.parametrize("cfg", range(NCFG))
@pytest.mark.parametrize("splits", [1, 3])
def test_gemm_every_tile_config(dev, cfg, splits):
    """Every tile config, with and without split-K, on ragged M / N / K tails (K = 1000: the last k-step is partial
    and reads A's padding columns against W's zero padding). Wave-split-K and 8-wave configs reject split-K."""
    lib = _lib.load()
    assert lib.mx_gemm_ncfg() == NCFG
    M, K, N = 300, 1000, 1152 + 68
    g = gen(cfg)
    x = torch.randn(M, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    ref = x.float() @ w.float().t() + b.float()
    lin = ops.MxLin(w, b)
    lin.cfgs[M] = (cfg, splits)
    print(f"gemm cfg={cfg} splits={splits}", flush=True)
    if splits > 1 and (lib.mx_gemm_cfg_kind(cfg) == 1 or cfg in NO_PSUM or cfg in KH2):
        with pytest.raises(_lib.MxError, match="-3"):
            lin(x.to(dev))
        return
    y = lin(x.to(dev))
    assert rel(y, ref) < 5e-3
    y2 = lin(x.to(dev))  # counters re-armed: a second call gives the same bits
    assert torch.equal(y.cpu(), y2.cpu())


@pytest.mark.parametrize("M,K,N", [(729, 1152, 1152), (729, 4304, 1152), (300, 1000, 1220)])
def test_gemm_partial_splits(dev, M, K, N):
    """mx_gemm_bf16_partial, every 4-wave config x 1-3 splits: the in-order fp32 sum of the partials is the fp32
    product to accumulation accuracy (K = 1000: the last k-step is partial). Configs without a partial-sum mode are
    rejected."""
    g = gen(M + K)
    x = torch.randn(M, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    ref = x.double() @ w.double().t()
    lin = ops.MxLin(w, None)
    lib = _lib.load()
    x2 = x.to(dev)
    for cfg in range(lib.mx_gemm_ncfg()):
        for sp in (1, 2, 3):
            P = torch.full((sp, M, N), float("nan"), device=dev)
            rc = ops._partial(lin, cfg, sp, x2, P, M)
            if cfg in NO_PSUM:  # their fp32 staging tile does not fit the LDS
                assert rc == -1
                continue
            assert rc == 0, (cfg, sp, rc)
            Pc = P.cpu()
            acc = Pc[0].clone()
            for i in range(1, sp):
                acc += Pc[i]
            err = (acc.double() - ref).abs().max().item()
            print(f"partial cfg={cfg} splits={sp} err={err:.2e}", flush=True)
            assert err <= 1e-5 * ref.abs().max().item(), (cfg, sp, err)


@pytest.mark.parametrize("cfg", [0, 3, 6, 8, 12, 19, 22])
def test_gemm_reduce_one_split_equals_fused(dev, cfg):
    """mx_gemm_reduce over one split of raw partials applies the fused kernel's epilogue to the same fp32
    accumulator: bit for bit mx_gemm_bf16 for act 0 / 1 / 2, the column-limited GELU, the residual (also
    row-broadcast) and the gated GELU; M = 63 and N = 4300 leave partial tiles."""
    M, K, N = 63, 1000, 4300
    g = gen(21)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    r = torch.randn(M, N, generator=g).to(BF).to(dev)
    r7 = torch.randn(7, N, generator=g).to(BF).to(dev)
    lin = ops.MxLin(w, b)
    x2 = ops._rows(x, lin.K)
    print(f"reduce cfg={cfg}", flush=True)
    for kw in (dict(), dict(gelu=True), dict(act="erf"), dict(gelu=True, act_cols=1000), dict(res=r),
               dict(gelu=True, res=r), dict(res=r7), dict(act="glu")):
        lin.cfgs[M] = (cfg, 1)
        y1 = lin(x, **kw).cpu()
        lin.cfgs[M] = (cfg, -1)
        y2 = lin(x, **kw).cpu()
        assert torch.equal(y1, y2), (cfg, kw)


@pytest.mark.parametrize("M,K,N", [(32, 8192, 2048), (64, 2048, 6144), (37, 2048, 2048), (730, 8192, 2048)])
def test_gemm_partial_reduce_splits_vs_fp32(dev, M, K, N):
    """The fence-free split-K (partial GEMM + mx_gemm_reduce, picks (cfg, -S)) at the prompt / query shapes: within
    the GEMM tolerance of fp32 for S = 2, 4, 8, 16 (with and without the residual), and without the residual within
    what a different fp32 summation order allows of the one-split result: one bf16 rounding of each plus
    K 2^-24 sum_k |x_k w_k| per element (the two differ only in that order; the rounding flips it causes are a few
    percent of the elements)."""
    g = gen(M + N)
    x = torch.randn(M, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    r = torch.randn(M, N, generator=g).to(BF)
    ref = x.float() @ w.float().t() + b.float()
    lin = ops.MxLin(w, b)
    xd, rd = x.to(dev), r.to(dev)
    lin.cfgs[M] = (6, 1)
    y1 = lin(xd).cpu().float()
    absum = x.float().abs() @ w.float().abs().t()
    slack = K * 2.0 ** -24 * absum + 2.0 ** -8 * y1.abs() * 2
    for S in (2, 4, 8, 16):
        for cfg in (6, 22, 0):
            lin.cfgs[M] = (cfg, -S)
            y = lin(xd).cpu()
            assert rel(y, ref) < 5e-3, (cfg, S)
            assert bool(((y.float() - y1).abs() <= slack).all()), (cfg, S)
            yr = lin(xd, res=rd).cpu()
            assert rel(yr, ref + r.float()) < 5e-3, (cfg, S)


def test_residual_layernorm_matches_unfused(dev):
    """x = bf16(bf16(sum P + bias) + res) bit for bit from the partials (CPU restatement, same fp32 order); the same
    within one ulp of the pre-rounding sum plus one of x of the single-pass GEMM epilogue (different summation order);
    y equals layernorm(x) exactly."""
    M, K, N = 729, 1152, 1152
    g = gen(11)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    r = (torch.randn(M, N, generator=g) * 4).to(BF).to(dev)
    gam = (1 + 0.1 * torch.randn(N, generator=g)).to(BF).to(dev)
    bet = (0.1 * torch.randn(N, generator=g)).to(BF).to(dev)
    lin = ops.MxLin(w, b)
    P = lin.partial(x)
    xo, yo = ops.residual_layernorm(P, lin.b, r, (gam, bet), eps=1e-6)
    xo2, none = ops.residual_layernorm(P, lin.b, r, None, eps=1e-6)
    assert none is None and torch.equal(xo.cpu(), xo2.cpu())
    Pc = P.cpu()
    acc = Pc[0].clone()
    for i in range(1, Pc.shape[0]):
        acc += Pc[i]
    gsum = acc + lin.b.cpu().float()
    exp = (gsum.to(BF).float() + r.cpu().float()).to(BF)
    assert torch.equal(xo.cpu(), exp)
    # Another summation order may round bf16(g) one ulp the other way; after + res that is one ulp of g plus one ulp
    # of the sum, which exceeds one ulp of the sum where g and res cancel.
    a, f = xo.float().cpu(), lin(x, res=r).float().cpu()
    tol = 2.0 ** -7 * (gsum.abs() + torch.maximum(a.abs(), f.abs())) + 1e-30
    over, frac = int(((a - f).abs() > tol).sum()), (a != f).float().mean().item()
    assert over == 0 and frac <= 1e-2, (P.shape[0], over, frac)
    assert torch.equal(yo.cpu(), ops.layernorm(xo, gam, bet, eps=1e-6).cpu())


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_residual_rmsnorm_matches_oracle(dev, splits):
    """mx_residual_rmsnorm on TRecViT's down / mlp3 shape (1280 x 768, K = 3072): x = bf16(bf16(sum P + bias) + res)
    bit for bit against the CPU restatement of the partials in split order; y against the oracle's RMSNorm chain
    (pack8.py:222-229) applied to that x: at most one bf16 ulp anywhere (its fp32 sum of the rounded squares runs in
    another order), on at most 1 % of the elements, and the rmsnorm kernel on the same x exactly."""
    import oracle.trecvit as otr
    M, K, N = 1280, 3072, 768
    g = gen(31 + splits)
    a = torch.randn(M, K, generator=g).to(BF).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF).to(dev)
    b = (torch.randn(N, generator=g) * 0.02).to(dev)
    r = (torch.randn(M, N, generator=g) * 2).to(BF).to(dev)
    scale = (torch.randn(N, generator=g) * 0.3).to(BF)
    sc1 = (scale.float() + 1).to(BF).to(dev)
    kt = K // 64
    P = torch.empty(splits, M, N, device=dev)
    _lib.call("mx_gemm_bf16_partial", _lib.stream(), 0, splits, a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
              P.data_ptr(), N, M * N, M, N, K, K)
    print(f"residual rmsnorm, {splits} splits of {kt} k-steps", flush=True)
    xo, yo = ops.residual_rmsnorm(P, b, r, sc1, eps=1e-6)
    Pc = P.cpu()
    acc = Pc[0].clone()
    for i in range(1, splits):
        acc += Pc[i]
    exp = ((acc + b.cpu()).to(BF).float() + r.cpu().float()).to(BF)
    assert torch.equal(xo.cpu(), exp)
    ref = otr.rmsnorm(exp, scale)
    d = (yo.cpu().view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert d.max().item() <= 1 and (d > 0).float().mean().item() <= 1e-2
    assert torch.equal(yo.cpu(), ops.rmsnorm(xo, sc1, eps=1e-6).cpu())
    full = (a.float() @ w.float().t()).cpu()
    assert rel(acc, full) < 1e-5  # the partials cover the whole K range


@pytest.mark.parametrize("M,K,N", [(729, 1152, 1152), (729, 4304, 1152), (100, 1152, 1152), (1280, 768, 768)])
def test_gemm_res_ln_matches_unfused(dev, M, K, N):
    """mx_gemm_bf16_res_ln (residual Linear + LayerNorm in one launch, row statistics exchanged between the tiles of
    a row block): x' within one ulp of the pre-rounding sum plus one of x' of the CPU restatement (another summation
    order than the CPU's, as test_residual_layernorm_matches_unfused); y within one bf16 ulp (of the largest operand
    of its last step) of the row LayerNorm kernel applied to the same x' (statistics summed in another order), on at
    most 0.1 % of the elements, and as close to an fp32 LayerNorm as that
    kernel's output (its bf16 rounding, ~1.5e-3 rel-L2, within 5 %). Three calls
    in a row with new inputs (each launch takes new epochs from the row blocks' generation counters), no timeout.
    Shapes: the batch-1 vision projection (and a 4304-deep K, and a 100-row grid) and TRecViT's attention
    out-projection with ln_2 over one frame (1280 x 768: 20 x 12 tiles)."""
    g = gen(M + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    gam = (1 + 0.1 * torch.randn(N, generator=g)).to(BF).to(dev)
    bet = (0.1 * torch.randn(N, generator=g)).to(BF).to(dev)
    lin = ops.MxLin(w, b)
    assert ops.res_ln_fits(M, N, dev)
    ws = ops.RlnWorkspace.get(dev, N)
    for call in range(3):
        x = torch.randn(M, K, generator=g).to(BF).to(dev)
        r = (torch.randn(M, N, generator=g) * 4).to(BF).to(dev)
        print(f"res_ln M={M} K={K} N={N} call {call}", flush=True)
        xo, yo = lin.res_ln(x, r, (gam, bet), eps=1e-6)
        torch.cuda.synchronize()
        assert ws.error() == 0
        gsum = x.cpu().float() @ w.float().t() + lin.b.cpu().float()
        exp = (gsum.to(BF).float() + r.cpu().float()).to(BF)
        a, f = xo.float().cpu(), exp.float()
        tol = 2.0 ** -7 * (gsum.abs() + torch.maximum(a.abs(), f.abs())) + 1e-30
        over, frac = int(((a - f).abs() > tol).sum()), (a != f).float().mean().item()
        assert over == 0 and frac <= 2e-2, (over, frac)
        y_row = ops.layernorm(xo, gam, bet, eps=1e-6)
        y32 = F.layer_norm(xo.float().cpu(), (N,), gam.float().cpu(), bet.float().cpu(), eps=1e-6)
        # one bf16 ulp of the largest operand of y = t + beta, t = (x' - mean) rstd gamma: where beta cancels t, a
        # last-bit change of the statistics moves a tiny y by more than one of its own ulps
        yb, yr, bb = yo.float().cpu(), y_row.float().cpu(), bet.float().cpu().expand(M, N)
        scale = torch.maximum(torch.maximum(yb.abs(), yr.abs()), torch.maximum(bb.abs(), (y32 - bb).abs()))
        assert bool(((yb - yr).abs() <= 2.0 ** -7 * scale + 1e-30).all()), (yb - yr).abs().max().item()
        assert (yb != yr).float().mean().item() <= 1e-3
        assert rel(yo, y32) <= 1.05 * rel(y_row, y32) + 1e-5, (rel(yo, y32), rel(y_row, y32))


def test_gemm_res_ln_interleaved_widths(dev):
    """Calls of different N and M in one process: (729, 1152), (100, 2048), (729, 1152), (100, 2048). Each N has
    its own statistics words (the tiles per row block decide where a row block's words sit, so words left by another
    N could carry an expected epoch); every call's x' is the unfused residual sum of its own inputs bit for bit
    (k loop of the same tile) and y within the row LayerNorm tolerance, with no timeout."""
    g = gen(77)
    lins = {}
    for call, (M, N) in enumerate([(729, 1152), (100, 2048), (729, 1152), (100, 2048)]):
        if N not in lins:
            w = (torch.randn(N, 1152, generator=g) * 0.02).to(BF)
            lins[N] = (ops.MxLin(w, (torch.randn(N, generator=g) * 0.02).to(BF)),
                       (1 + 0.1 * torch.randn(N, generator=g)).to(BF).to(dev), (0.1 * torch.randn(N, generator=g)).to(BF).to(dev))
        lin, gam, bet = lins[N]
        assert ops.res_ln_fits(M, N, dev)
        x = torch.randn(M, 1152, generator=g).to(BF).to(dev)
        r = (torch.randn(M, N, generator=g) * 4).to(BF).to(dev)
        print(f"res_ln interleaved call {call}: M={M} N={N}", flush=True)
        xo, yo = lin.res_ln(x, r, (gam, bet), eps=1e-6)
        xs, ys = ops.residual_layernorm(lin.partial(x), lin.b, r, (gam, bet), eps=1e-6)
        torch.cuda.synchronize()
        assert ops.RlnWorkspace.device_error(dev) == 0
        gsum = x.cpu().float() @ lins[N][0].w[:, :1152].cpu().float().t() + lin.b.cpu().float()
        a, f = xo.float().cpu(), xs.float().cpu()
        tol = 2.0 ** -7 * (gsum.abs() + torch.maximum(a.abs(), f.abs())) + 1e-30
        assert int(((a - f).abs() > tol).sum()) == 0, call
        y_row = ops.layernorm(xo, gam, bet, eps=1e-6).float().cpu()
        scale = torch.maximum(y_row.abs(), bet.float().cpu().abs().expand(M, N)) + y_row.abs()
        assert bool(((yo.float().cpu() - y_row).abs() <= 2.0 ** -7 * scale + 1e-30).all()), call
        assert (yo.float().cpu() != y_row).float().mean().item() <= 1e-3, call


@pytest.mark.parametrize("M", [1280, 100])
def test_gemm_res_rms_matches_unfused(dev, M):
    """mx_gemm_bf16_res_rms (residual Linear + the TRecViT RMSNorm in one launch) on TRecViT's linear_out shape
    (M x 768, K = 768; a frame is 1280 rows, 20 x 12 tiles): x' within one ulp of the pre-rounding sum plus one of
    the CPU restatement's x' (as the LayerNorm form); y against the oracle's RMSNorm chain (pack8.py:222-229) applied
    to that x': at most one bf16 ulp anywhere, on at most 1 % of the elements (the tiles' fp32 sums of the rounded
    squares run in another order than the oracle's). Each call alternates with the LayerNorm form on the same
    statistics words (same N), which must give the same x' bit for bit (one kernel k loop); three of each, no
    timeout."""
    import oracle.trecvit as otr
    N = K = 768
    g = gen(501 + M)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    lin = ops.MxLin(w, b)
    scale = (torch.randn(N, generator=g) * 0.3).to(BF)
    sc1 = (scale.float() + 1).to(BF).to(dev)
    gam = (1 + 0.1 * torch.randn(N, generator=g)).to(BF).to(dev)
    bet = (0.1 * torch.randn(N, generator=g)).to(BF).to(dev)
    assert ops.res_ln_fits(M, N, dev)
    for call in range(3):
        x = torch.randn(M, K, generator=g).to(BF).to(dev)
        r = (torch.randn(M, N, generator=g) * 2).to(BF).to(dev)
        print(f"res_rms M={M} call {call}", flush=True)
        xo, yo = lin.res_rms(x, r, sc1, eps=1e-6)
        xl, _ = lin.res_ln(x, r, (gam, bet), eps=1e-6)
        torch.cuda.synchronize()
        assert ops.RlnWorkspace.device_error(dev) == 0
        assert torch.equal(xl, xo)
        gsum = x.cpu().float() @ w.float().t() + lin.b.cpu().float()
        exp = (gsum.to(BF).float() + r.cpu().float()).to(BF)
        a, f = xo.float().cpu(), exp.float()
        tol = 2.0 ** -7 * (gsum.abs() + torch.maximum(a.abs(), f.abs())) + 1e-30
        assert int(((a - f).abs() > tol).sum()) == 0, call
        ref = otr.rmsnorm(xo.cpu(), scale)
        d = (yo.cpu().view(torch.int16).int() - ref.view(torch.int16).int()).abs()
        assert d.max().item() <= 1 and (d > 0).float().mean().item() <= 1e-2, (d.max().item(), (d > 0).float().mean())
        y_row = ops.rmsnorm(xo, sc1, eps=1e-6)
        assert (yo != y_row).float().mean().item() <= 1e-2


def test_gemm_res_ln_refuses_a_grid_larger_than_the_gpu(dev):
    """Two crops (1458 rows: 23 x 18 tiles > 256 CUs) cannot all be resident: refused before launching."""
    lin = ops.MxLin(torch.zeros(1152, 1152, dtype=BF), torch.zeros(1152))
    x = torch.zeros(1458, 1152, dtype=BF, device=dev)
    ln = (torch.ones(1152, dtype=BF, device=dev), torch.zeros(1152, dtype=BF, device=dev))
    assert not ops.res_ln_fits(1458, 1152, dev)
    with pytest.raises(_lib.MxError, match="-2"):
        lin.res_ln(x, x, ln)


@pytest.mark.parametrize("cfg", [None, 0, 19])
def test_gelu_epilogues_every_bf16_input(dev, cfg):
    """The GELU epilogues (erf: a Chebyshev erfc fit; tanh: x / (1 + exp(-2u))) on every finite bf16 value in
    [-12, 12]: an identity weight makes the linear output the input itself, so each value goes through the epilogue
    once. Against torch's F.gelu in fp32 (tgemm.py:21-25 for tanh; nn.GELU for erf): for x >= -4, within two bf16
    ulps and at most 0.5 % of the values differing at all (torch's own erf / tanh and the hardware exp2 / reciprocal
    each round differently in the last fp32 bit); below, where torch's 1 + erf / 1 + tanh cancels and its result
    carries fp32 noise of ~|x| 6e-8, within 2e-6 absolute (those outputs are below 1.3e-4)."""
    allv = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(BF)
    vals = allv[torch.isfinite(allv.float()) & (allv.float().abs() <= 12)]
    K = 1024
    M = (vals.numel() + K - 1) // K
    x = torch.zeros(M * K, dtype=BF)
    x[:vals.numel()] = vals
    x = x.view(M, K)
    lin = ops.MxLin(torch.eye(K, dtype=BF), torch.zeros(K, dtype=BF))
    if cfg is not None:
        lin.cfgs[M] = (cfg, 1)
    print(f"gelu every bf16 cfg={cfg} values={vals.numel()}", flush=True)
    xd = x.to(dev)
    assert torch.equal(lin(xd).cpu(), x)  # the identity linear passes every value through unchanged
    xf = x.float()
    core = xf >= -4.0
    for kw, ref in ((dict(act="erf"), F.gelu(xf)), (dict(gelu=True), F.gelu(xf, approximate="tanh"))):
        y = lin(xd, **kw).cpu()
        exp = ref.to(BF)
        assert within_ulps(y[core], exp[core], n=2, frac=5e-3), kw
        assert ((y[~core].float() - exp[~core].float()).abs() <= 2e-6).all(), kw


@pytest.mark.parametrize("cfg", [None, 0, 7, 8, 12, 15, 16, 17])
def test_gemm_epilogues_match_unfused(dev, cfg):
    """GELU applied to the bf16-rounded linear output, then + residual (md2fast.py:55-67; i8gemm.hip:378); the gated
    GELU of interleaved (gate, up) columns and the column-limited activation; per tile config (None: the tuned one),
    N = 4300 leaves a partial last column tile and an 8-column chunk with 4 valid columns."""
    M, K, N = 729, 1152, 4300
    g = gen(3)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    r = torch.randn(M, N, generator=g).to(BF).to(dev)
    lin = ops.MxLin(w, b)
    if cfg is not None:
        lin.cfgs[M] = (cfg, 1)
    print(f"epilogues cfg={cfg}", flush=True)
    y0 = lin(x).cpu()
    y_g = lin(x, act="glu").cpu()
    exp_g = (F.gelu(y0[:, 0::2].float(), approximate="tanh").to(BF).float() * y0[:, 1::2].float()).to(BF)
    assert y_g.shape == (M, N // 2) and within_ulps(y_g, exp_g)
    y_c = lin(x, gelu=True, act_cols=1024).cpu()
    assert torch.equal(y_c[:, 1024:], y0[:, 1024:])
    assert within_ulps(y_c[:, :1024], F.gelu(y0[:, :1024].float(), approximate="tanh").to(BF))
    y_t = lin(x, gelu=True).cpu()
    y_e = lin(x, act="erf").cpu()
    y_r = lin(x, res=r).cpu()
    y_tr = lin(x, gelu=True, res=r).cpu()
    # the same op sequence on the CPU from the kernel's own bf16 linear output; GELU's fp32 tanh/erf may differ
    # from the CPU's by an fp32 ulp, which can move a result by one bf16 ulp
    assert within_ulps(y_t, F.gelu(y0.float(), approximate="tanh").to(BF))
    assert within_ulps(y_e, F.gelu(y0.float()).to(BF))
    assert torch.equal(y_r, (y0.float() + r.cpu().float()).to(BF))
    exp_tr = (F.gelu(y0.float(), approximate="tanh").to(BF).float() + r.cpu().float()).to(BF)
    assert within_ulps(y_tr, exp_tr, n=2)


def test_gemm_residual_row_broadcast(dev):
    """r_rows: a (T, N) table added to every T-row slab of the output (the position embedding)."""
    T, B, K, N = 729, 3, 592, 1152
    g = gen(5)
    x = torch.randn(B * T, K, generator=g).to(BF).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    pos = torch.randn(T, N, generator=g).to(BF).to(dev)
    lin = ops.MxLin(w, None)
    y = lin(x, res=pos).cpu()
    y0 = lin(x).cpu()
    assert torch.equal(y, (y0.float() + pos.cpu().float().repeat(B, 1)).to(BF))


def _sdpa_ref(q, k, v, scale, mask=None):
    q, k, v = q.float().cpu(), k.float().cpu(), v.float().cpu()
    s = (q @ k.transpose(-1, -2)) * scale
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    return torch.softmax(s, dim=-1) @ v


@pytest.mark.parametrize("B,H,T,D", [(1, 16, 729, 72), (2, 16, 729, 72), (1, 12, 1280, 64), (1, 32, 730, 64), (1, 4, 33, 72),
                                     (6, 16, 729, 72), (5, 12, 1280, 64)])
def test_sdpa_strided_views(dev, B, H, T, D):
    """q, k, v as strided views of a fused qkv output (the vision layout, md2fast.py:154)."""
    g = gen(B * 100 + T)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(BF)
    q, k, v = [t.view(B, T, H, D).transpose(1, 2) for t in qkv.chunk(3, dim=-1)]
    ref = _sdpa_ref(q, k, v, D ** -0.5).transpose(1, 2).reshape(B, T, H * D)
    qd = qkv.to(dev)
    q2, k2, v2 = [t.view(B, T, H, D).transpose(1, 2) for t in qd.chunk(3, dim=-1)]
    print(f"sdpa B={B} H={H} T={T} D={D}", flush=True)
    out = ops.sdpa(q2, k2, v2)
    assert out.shape == (B, T, H * D)
    assert rel(out, ref) < 1e-2
    assert (out.float().cpu() - ref).abs().max().item() < 5e-2


def test_sdpa_prefix_causal_mask(dev):
    """Prompt prefill mask (md2fast.py:132-136): prompt row i sees all prefix keys and prompt keys <= i."""
    H, P, L, D = 32, 730, 64, 64
    g = gen(11)
    kc = torch.randn(1, H, P + L, D, generator=g).to(BF)
    vc = torch.randn(1, H, P + L, D, generator=g).to(BF)
    q = torch.randn(1, H, L, D, generator=g).to(BF)
    m = torch.zeros(L, P + L, dtype=torch.bool)
    m[:, :P] = True
    m[:, P:] = torch.tril(torch.ones(L, L, dtype=torch.bool))
    ref = _sdpa_ref(q, kc, vc, 0.125, m[None, None]).transpose(1, 2).reshape(1, L, H * D)
    out = ops.sdpa(q.to(dev), kc.to(dev), vc.to(dev), qpos0=P, causal_from=P)
    assert rel(out, ref) < 1e-2
    # a plain causal self-attention, too
    T = 200
    q3 = torch.randn(1, 8, T, 64, generator=g).to(BF)
    cm = torch.tril(torch.ones(T, T, dtype=torch.bool))
    ref3 = _sdpa_ref(q3, q3, q3, 0.125, cm[None, None]).transpose(1, 2).reshape(1, T, 512)
    qd = q3.to(dev)
    out3 = ops.sdpa(qd, qd, qd, causal_from=0)
    assert rel(out3, ref3) < 1e-2


@pytest.mark.parametrize("B,L", [(3, 96), (6, 96)])
def test_sdpa_batched_query_mask(dev, B, L):
    """The batched yes/no query's mask (every question sees the 730-token prefix and its own ids causally) at a grid
    size served by 8-wave (B = 3) and 16-wave (B = 6) workgroups."""
    H, P, D = 32, 730, 64
    g = gen(13 + B)
    kc = torch.randn(B, H, P + L, D, generator=g).to(BF)
    vc = torch.randn(B, H, P + L, D, generator=g).to(BF)
    q = torch.randn(B, H, L, D, generator=g).to(BF)
    m = torch.zeros(L, P + L, dtype=torch.bool)
    m[:, :P] = True
    m[:, P:] = torch.tril(torch.ones(L, L, dtype=torch.bool))
    ref = _sdpa_ref(q, kc, vc, 0.125, m[None, None]).transpose(1, 2).reshape(B, L, H * D)
    print(f"sdpa masked query B={B} L={L}", flush=True)
    out = ops.sdpa(q.to(dev), kc.to(dev), vc.to(dev), qpos0=P, causal_from=P)
    assert rel(out, ref) < 1e-2
    assert (out.float().cpu() - ref).abs().max().item() < 5e-2


@pytest.mark.parametrize("rows,D", [(729, 1152), (1458, 1152), (730, 2048), (1, 2048), (1280, 768)])
def test_layernorm(dev, rows, D):
    g = gen(rows + D)
    x = (torch.randn(rows, D, generator=g) * 3 + 1).to(BF)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
    b = (0.1 * torch.randn(D, generator=g)).to(BF)
    ref = F.layer_norm(x.float(), (D,), w.float(), b.float(), 1e-5)
    y = ops.layernorm(x.to(dev), w.to(dev), b.to(dev), eps=1e-5)
    assert rel(y, ref) < 4e-3
    # one rounding of the fp32 result: at most 1 ulp away
    assert ((y.float().cpu() - ref).abs() <= ref.abs() * 2 ** -8 + 1e-6).float().mean().item() > 0.999


def test_patchify_matches_oracle(dev):
    import oracle.md2_vision as ov
    img = torch.randint(0, 256, (2, 378, 378, 3), generator=gen(1), dtype=torch.uint8)
    ref = ov.normalize_patchify(img).reshape(2 * 729, 588)
    y = ops.patchify(img.to(dev), 14, mode=0, ldo=592).cpu()
    assert torch.equal(y[:, :588], ref)
    assert torch.count_nonzero(y[:, 588:]) == 0
