"""The reference-side binding (strix_halo_maxx_amd.refbind, the module a maintainer adds next to hgemm.py) driven
through the reference's own dataflow: the oracle's operator-injected tower (oracle.md2_vision.tower_with, the
FastMD2._vision loop of md2fast.py:147-160 with lin_cls / hattn plugged in, md2fast.py:71, 87-94) runs with
linear_cls = refbind.MxLin and attention_cls = refbind.Attn, with the residual adds fused into the GEMM epilogue and
without (USE_FUSED_RES, md2fast.py:51), against the oracle's all-torch tower; and refbind.MxI8Lin (the HI8Lin
protocol) against the oracle's W8A8 restatement bit for bit.
Tolerances as in the vision tests: end to end (27 blocks + post-LN) rel-L2 <= 2e-2."""
import pytest
import torch

import oracle.md2_text as ot
import oracle.md2_vision as ov
import strix_halo_maxx_amd.refbind as rb
import strix_halo_maxx_amd.synth as S

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("fused_res", [True, False])
def test_reference_dataflow_tower_with_refbind(dev, fused_res):
    w = S.vision_weights(0)
    img = S.images_u8(1, 1)
    ref = ov.tower(w, img)[0]
    print(f"refbind tower, fused residual {fused_res}", flush=True)
    out = ov.tower_with(w, img[0].to(dev), rb.MxLin, rb.Attn, device=dev, fuse_res=fused_res)
    r = rel(out, ref)
    print(f"refbind tower, fused residual {fused_res}: rel-L2 vs oracle {r:.2e}", flush=True)
    assert out.shape == (729, 1152) and out.device.type == "cuda"
    assert r <= 2e-2


def test_refbind_w8a8_linear_protocol(dev):
    """refbind.MxI8Lin against the oracle's W8A8 restatement (hgemm.py:95-137): quant() and the plain output bit for
    bit, the shared quantisation (pre=) equal to quantising again, the fused residual equal to the separate bf16 add,
    GELU within one bf16 ulp (plus 1e-6 absolute where 1 + tanh cancels) on at most 2 % of the elements (it acts on
    the unrounded fp32 value, so the hardware tanh's error moves a few roundings)."""
    g = torch.Generator().manual_seed(5)
    M, K, N = 64, 2048, 6144
    x = torch.randn(M, K, generator=g).to(BF)
    W = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    r = torch.randn(M, N, generator=g).to(BF)
    lin = rb.MxI8Lin(W.to(dev), b.to(dev), BF)
    xd = x.to(dev)
    q, s = lin.quant(xd)
    qr, sr = ot.quant_rows(x)
    assert torch.equal(q.cpu(), qr) and torch.equal(s.cpu(), sr)
    wq, sw = ot.quant_weight(W)
    ref = ot.i8_linear(qr, sr, wq, sw, b)
    y = lin(xd)
    assert torch.equal(y.cpu(), ref)
    assert torch.equal(lin(xd, pre=(q, s)).cpu(), ref)
    assert torch.equal(lin(xd, res=r.to(dev)).cpu(), (ref + r))
    yg = lin(xd, gelu=True).cpu()
    refg = ot.i8_linear(qr, sr, wq, sw, b, gelu_tanh=True)
    d = (yg.float() - refg.float()).abs()
    assert bool((d <= 2.0 ** -7 * refg.float().abs() + 1e-6).all())
    assert (d > 0).float().mean().item() <= 0.02
