"""The reference-side binding (strix_halo_maxx_amd.refbind, the module a maintainer adds next to hgemm.py) driven
the way the reference drives its own op classes: a `_vision` loop shaped exactly like FastMD2._vision
(moondream/gpu/md2fast.py:147-160, with _ln / gelu / mlp / lin_res of md2fast.py:43-67 restated below as the
harness) with lin_cls = refbind.MxLin and hattn = refbind.Attn, in both USE_FUSED_RES settings, against the oracle's
tower; and refbind.MxI8Lin (the HI8Lin protocol) against the oracle's W8A8 restatement bit for bit.
Tolerances as in the vision tests: end to end (27 blocks + post-LN) rel-L2 <= 2e-2."""
import pytest
import torch
import torch.nn.functional as F

import oracle.md2_text as ot
import oracle.md2_vision as ov
import strix_halo_maxx_amd.refbind as rb
import strix_halo_maxx_amd.synth as S

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
GRID, PATCH, NTOK = 27, 14, 729


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


# ---- the reference's helpers (md2fast.py:43-67), as the harness the op classes plug into
class Flags:
    USE_FUSED_RES = False


def _ln(x, wb):
    return F.layer_norm(x, (x.shape[-1],), wb[0], wb[1])


def gelu(x):
    return F.gelu(x, approximate="tanh")


def mlp(fc1, fc2, h, res=None, pre=None):
    kw = {"pre": pre} if pre is not None else {}
    a = fc1(h, gelu=True, **kw) if getattr(fc1, "fused_gelu", False) else gelu(fc1(h, **kw))
    if res is not None and Flags.USE_FUSED_RES and getattr(fc2, "fused_res", False):
        return fc2(a, res=res)
    out = fc2(a)
    return out if res is None else out + res


def lin_res(l, x, res):
    if Flags.USE_FUSED_RES and getattr(l, "fused_res", False):
        return l(x, res=res)
    return l(x) + res


class RefShapedVision:
    """FastMD2's vision half with `lin_cls` and `hattn` plugged in (md2fast.py:87-94, 147-157)."""

    def __init__(self, w, lin_cls, attn_cls, dev, H=16):
        g = lambda n: w[n].to(dev)
        L = lambda n: lin_cls(g(n + ".weight"), g(n + ".bias"), BF)
        self.patch_emb, self.pos_emb = L("patch_emb"), g("pos_emb")
        n = 0
        while f"blocks.{n}.ln1.weight" in w:
            n += 1
        self.vblocks = [dict(ln1=(g(f"blocks.{i}.ln1.weight"), g(f"blocks.{i}.ln1.bias")), qkv=L(f"blocks.{i}.attn.qkv"),
                             proj=L(f"blocks.{i}.attn.proj"),
                             ln2=(g(f"blocks.{i}.ln2.weight"), g(f"blocks.{i}.ln2.bias")),
                             fc1=L(f"blocks.{i}.mlp.fc1"), fc2=L(f"blocks.{i}.mlp.fc2")) for i in range(n)]
        self.post_ln = (g("post_ln.weight"), g("post_ln.bias"))
        self.vh = H
        self.attn_v = attn_cls(H, NTOK, 1152 // H)

    def _vision(self, img_u8):
        x = img_u8.permute(2, 0, 1)[None].to(BF).div_(255.0).sub_(0.5).div_(0.5)
        x = x.reshape(1, 3, GRID, PATCH, GRID, PATCH).permute(0, 2, 4, 1, 3, 5).reshape(1, NTOK, 3 * PATCH * PATCH)
        x = self.patch_emb(x) + self.pos_emb
        H = self.vh
        for b in self.vblocks:
            h = _ln(x, b["ln1"])
            q, k, v = [t.view(1, NTOK, H, -1).transpose(1, 2) for t in b["qkv"](h).chunk(3, dim=-1)]
            a = self.attn_v(q, k, v)
            x = lin_res(b["proj"], a, x)
            x = mlp(b["fc1"], b["fc2"], _ln(x, b["ln2"]), res=x)
        return _ln(x, self.post_ln)[0]


@pytest.mark.parametrize("fused_res", [True, False])
def test_reference_shaped_vision_loop_with_refbind(dev, fused_res):
    w = S.vision_weights(0)
    img = S.images_u8(1, 1)
    ref = ov.tower(w, img)[0]
    m = RefShapedVision(w, rb.MxLin, rb.Attn, dev)
    Flags.USE_FUSED_RES = fused_res
    try:
        out = m._vision(img[0].to(dev))
    finally:
        Flags.USE_FUSED_RES = False
    r = rel(out, ref)
    print(f"reference-shaped _vision, USE_FUSED_RES={fused_res}: rel-L2 vs oracle {r:.2e}", flush=True)
    assert out.shape == (NTOK, 1152)
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
