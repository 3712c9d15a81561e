"""The allocation-free GEMM entry point (mx_gemm_bf16_noalloc) against mx_gemm_bf16 with a caller-allocated split-K
workspace, through the C ABI: bit for bit, on two calls in a row (the second smaller, so it reuses the fixed
workspace the first one left dirty), for in-kernel split-K and for the split-free path; a call whose split-K
workspace would exceed the fixed maximum is refused with the workspace status before anything is launched."""
import pytest
import torch

from strix_halo_maxx_amd import _lib

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    Kw = (K + 63) // 64 * 64
    A = torch.randn(M, K, generator=g).to(BF)
    W = torch.zeros(N, Kw, dtype=BF)
    W[:, :K] = (torch.randn(N, K, generator=g) * 0.05).to(BF)
    b = torch.randn(N, generator=g) * 0.1
    R = torch.randn(M, N, generator=g).to(BF)
    return A, W, b, R, Kw


def _gemm(dev, fn, cfg, splits, A, W, b, R, K, Kw, act):
    M, N = A.shape[0], W.shape[0]
    Ad, Wd, bd, Rd = A.to(dev), W.to(dev), b.to(dev), R.to(dev)
    C = torch.full((M, N), float("nan"), device=dev).to(BF)
    args = [_lib.stream(), cfg, splits, Ad.data_ptr(), K, Wd.data_ptr(), Kw, bd.data_ptr(), Rd.data_ptr(), N, 0,
            C.data_ptr(), N, M, N, K, Kw, act, 0]
    if fn == "mx_gemm_bf16":
        lib = _lib.load()
        ne, nc = lib.mx_gemm_ws_elems(cfg, splits, M, N), lib.mx_gemm_ws_counters(cfg, splits, M, N)
        ws = torch.empty(max(ne, 1), device=dev)
        cnt = torch.zeros(max(nc, 1), device=dev, dtype=torch.int32)
        args += [ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel()]
    _lib.call(fn, *args)
    torch.cuda.synchronize()
    return C.cpu()


@pytest.mark.parametrize("cfg,splits", [(0, 4), (3, 3), (8, 1)])
def test_noalloc_gemm_equals_workspace_gemm_twice(dev, cfg, splits):
    for M, N, K, act, seed in ((729, 1152, 4304, 1, 1), (300, 768, 1152, 0, 2)):
        print(f"noalloc cfg {cfg} splits {splits}: M {M} N {N} K {K} act {act}", flush=True)
        A, W, b, R, Kw = _operands(M, N, K, seed)
        ref = _gemm(dev, "mx_gemm_bf16", cfg, splits, A, W, b, R, K, Kw, act)
        out = _gemm(dev, "mx_gemm_bf16_noalloc", cfg, splits, A, W, b, R, K, Kw, act)
        assert not torch.isnan(ref.float()).any()
        assert torch.equal(out, ref)


def test_noalloc_gemm_refuses_beyond_its_workspace(dev):
    """A split whose partials exceed the fixed array is refused (-3) before any launch, on real operand buffers: the
    output keeps its NaN fill."""
    lib = _lib.load()
    M, N, Kw = 1024, 1024, 1152
    assert lib.mx_gemm_ws_elems(0, 8, M, N) > lib.mx_gemm_noalloc_max_ws()
    A = torch.zeros(M, Kw, device=dev, dtype=torch.bfloat16)
    W = torch.zeros(N, Kw, device=dev, dtype=torch.bfloat16)
    C = torch.full((M, N), float("nan"), device=dev, dtype=torch.bfloat16)
    rc = lib.mx_gemm_bf16_noalloc(_lib.stream(), 0, 8, A.data_ptr(), Kw, W.data_ptr(), Kw, None, None, 0, 0,
                                  C.data_ptr(), N, M, N, Kw, Kw, 0, 0)
    assert rc == -3
    torch.cuda.synchronize()
    assert bool(torch.isnan(C.float()).all())
