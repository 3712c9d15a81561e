"""SigLIP vision tower parity: the HIP path (VisionTower) vs the oracle's restatement of the reference's PyTorch bf16
path (oracle/md2_vision.py) on identical seeded weights and pixels.

Tolerances (stated for the floating-point hidden states): per block, given the same block input,
  * rel-L2 <= 1e-2;
  * elementwise |diff| <= 5e-2 + 2 bf16 ulps of the oracle value, and |diff| > 5e-2 on under 1e-3 of the elements;
  * no less accurate than the oracle itself: max |hip - fp32| <= 1.5 max |oracle - fp32| + 1e-2, where fp32 is the
    same block computed in fp32 from the same bf16 input and weights.
The ulp allowance exists because the residual stream grows past 4 and 8 in the later blocks (1.4 % of block 27's
elements exceed 8 at this seed), where the bf16 spacing is 0.03 / 0.06: the oracle's own bf16 result is up to 0.066
away from fp32 there, so two correct bf16 computations accumulating in different orders can differ by more than
5e-2. End to end (27 blocks + post-LN, errors compound), rel-L2 <= 2e-2."""
import pytest
import torch

import oracle.md2_vision as ov
import strix_halo_maxx_amd.md2 as md2
import strix_halo_maxx_amd.synth as S

pytestmark = pytest.mark.gpu
REL, MAXABS = 1e-2, 5e-2


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


def check(a, b):
    """(rel-L2, excess, frac_over, raw): excess = max(|a - b| - (5e-2 + 2 bf16 ulps of b)) (<= 0 when within
    tolerance), frac_over = fraction of elements with |a - b| > 5e-2, raw = max |a - b|."""
    a, b = a.float().cpu(), b.float().cpu()
    ulp = torch.where(b == 0, torch.zeros_like(b), torch.ldexp(torch.ones_like(b), torch.frexp(b)[1] - 8))
    d = (a - b).abs()
    excess = (d - (MAXABS + 2 * ulp)).max().item()
    return rel(a, b), excess, (d > MAXABS).float().mean().item(), d.max().item()


def ok(a, b):
    r, ex, fr, raw = check(a, b)
    return r <= REL and ex <= 0 and fr < 1e-3, (r, ex, fr, raw)


def rawmax(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


@pytest.fixture(scope="module")
def full():
    w = S.vision_weights(0)
    img = S.images_u8(1, 1)
    ref, hs = ov.tower(w, img, return_blocks=True)
    return w, img, ref, hs


def test_one_block_config0(dev):
    """Config 0: one block, x ~ N(0,1) (1, 729, 1152), weights N(0, 0.02), LN gamma 1 beta 0."""
    w = S.vision_weights(0, layers=1)
    x = S.activations(1, (1, 729, 1152))
    ref = ov.block(w, 0, x)
    vt = md2.VisionTower(w)
    y = vt.block(vt.blocks[0], x.view(729, 1152).to(dev), 1).view(1, 729, 1152)
    good, st = ok(y, ref)
    print("block0 (rel, excess, frac>5e-2, raw max-abs)", st, flush=True)
    assert good, st


def test_batch2_crops_independent(dev):
    """Batching crops stacks them as token rows; a crop's result must not depend on its batch neighbours. Changing
    crop 0 leaves crop 1's output bit-identical (same batch size, so the same kernels and tiles), and crop 1 batched
    agrees with crop 1 alone to the per-block tolerance (batch 1 and batch 2 may pick different GEMM tilings, whose
    summation orders can differ in the last bit)."""
    w = S.vision_weights(0, layers=1)
    x = S.activations(2, (2, 729, 1152))
    vt = md2.VisionTower(w)
    y2 = vt.block(vt.blocks[0], x.view(-1, 1152).to(dev), 2).view(2, 729, 1152).cpu()
    xb = x.clone()
    xb[0] = S.activations(3, (1, 729, 1152))[0]
    y2b = vt.block(vt.blocks[0], xb.view(-1, 1152).to(dev), 2).view(2, 729, 1152).cpu()
    assert torch.equal(y2[1], y2b[1])
    assert not torch.equal(y2[0], y2b[0])
    y1 = vt.block(vt.blocks[0], x[1].reshape(729, 1152).to(dev), 1).view(729, 1152).cpu()
    good, st = ok(y2[1], y1)
    assert good, st


def test_tower_per_block_and_end_to_end(dev, full):
    """Config 1, batch 1: every one of the 27 blocks within tolerance given the oracle's input to that block, and the
    whole tower (pixels -> post-LN features) within the end-to-end tolerance."""
    w, img, ref, hs = full
    vt = md2.VisionTower(w)
    emb = vt.embed(img.to(dev))
    good, st = ok(emb, hs[0][0])
    print("embed", st, flush=True)
    assert good, st
    worst = 0.0
    w32 = {k: v.float() for k, v in w.items()}
    for i, b in enumerate(vt.blocks):
        y = vt.block(b, hs[i][0].to(dev), 1)
        good, st = ok(y, hs[i + 1][0])
        worst = max(worst, st[0])
        assert good, (i, st)
        if i % 4 == 3 or i == len(vt.blocks) - 1:
            y32 = ov.block(w32, i, hs[i].float())[0]
            e_hip, e_ora = rawmax(y, y32), rawmax(hs[i + 1][0], y32)
            assert e_hip <= 1.5 * e_ora + 1e-2, (i, e_hip, e_ora)
    out = vt(img.to(dev))
    print("last block raw max-abs", rawmax(y, hs[-1][0]), flush=True)
    print("worst block rel", worst, "end-to-end rel", rel(out, ref), flush=True)
    assert rel(out, ref) <= 2e-2


def test_tower_batch13(dev, full):
    """Config 1, batch 13 (1 global + 12 local crops): every crop matches its own batch-1 oracle output."""
    w, _, _, _ = full
    imgs = S.images_u8(7, 13)
    vt = md2.VisionTower(w)
    out = vt(imgs.to(dev)).cpu()
    for i in (0, 6, 12):
        ref = ov.tower(w, imgs[i:i + 1])
        assert rel(out[i], ref[0]) <= 2e-2, i


def test_tower_batch256_config4(dev, full):
    """Config 4, the throughput-bound tower at batch 256 (186,624 token rows; the large-M GEMM tiles, not the
    split-K batch-1 path): the first, a middle and the last crop each match their own batch-1 oracle output."""
    w, _, _, _ = full
    imgs = S.images_u8(8, 256)
    vt = md2.VisionTower(w)
    out = vt(imgs.to(dev))
    assert out.shape == (256, 729, 1152)
    for i in (0, 131, 255):
        ref = ov.tower(w, imgs[i:i + 1])
        r = rel(out[i], ref[0])
        print(f"batch 256, crop {i}: rel-L2 vs oracle {r:.2e}", flush=True)
        assert r <= 2e-2, i
    del out
    torch.cuda.empty_cache()


def test_projection_mlp_vs_oracle(dev):
    """The post-LN features through cat([x, x]) -> fc1 2304 -> 8192 + GELU-tanh -> fc2 8192 -> 2048
    (md2fast.py:158-160; mlp md2fast.py:55-61): VisionTower.project on the oracle's post-LN features against the
    oracle's projection of the same features (rel-L2 <= 1e-2), and the whole tower with project=True against
    the oracle's tower(project=True) (the end-to-end bound, rel-L2 <= 2e-2)."""
    w = S.vision_weights(0, proj=True)
    img = S.images_u8(1, 1)
    feats = ov.tower(w, img)
    ref = ov.tower(w, img, project=True)
    assert ref.shape == (1, 729, 2048)
    vt = md2.VisionTower(w)
    p = vt.project(feats[0].to(dev))
    ref_p = ov.lin(ov.gelu(ov.lin(torch.cat([feats, feats], -1), w["proj_mlp.fc1.weight"], w["proj_mlp.fc1.bias"])),
                   w["proj_mlp.fc2.weight"], w["proj_mlp.fc2.bias"])
    assert torch.equal(ref_p, ref)
    r1 = rel(p, ref[0])
    out = vt(img.to(dev), project=True)
    r2 = rel(out, ref)
    print(f"projection on oracle features rel {r1:.2e}; tower + projection rel {r2:.2e}", flush=True)
    assert out.shape == (1, 729, 2048)
    assert r1 <= 1e-2 and r2 <= 2e-2


def test_graph_replay_bit_exact(dev, full):
    """HIP-graph replay of the ctypes-launched kernels equals eager bit for bit (test_hgemm.py:51-67), over
    several replays with eager work in between."""
    w, img, _, _ = full
    small = {k: v for k, v in w.items() if not k.startswith("blocks.") or int(k.split(".")[1]) < 3}
    vt = md2.VisionTower(small)
    buf = img.to(dev).clone()
    eager = vt(buf).clone()
    g, out = vt.capture(buf)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        vt(buf)  # eager work between replays
        torch.cuda.synchronize()
