"""Pins of the oracle (CPU, no GPU needed). The reference ships no golden vectors for this path (its regression files
davis_reg.npy / regress_*.npz / ref/baseline.json are referenced but absent), so each oracle function is checked
against what the mathematics fixes: closed forms, fp64 brute force on small inputs, invariants and special cases.
Each check is chosen so that a plausible restatement mistake (wrong eps, swapped GELU form, swapped rope halves,
missing residual, wrong scan operator order, wrong tap order) fails it."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.md2_text as ot
import oracle.md2_vision as ov
import oracle.trecvit as otr
import strix_halo_maxx_amd.synth as S

BF = torch.bfloat16


def bfr(x):
    return torch.as_tensor(x).to(BF).double()


def gen(s):
    return torch.Generator().manual_seed(s)


# ---------------------------------------------------------------------------------------------- shared ops
def test_layernorm_matches_closed_form_and_eps():
    """F.layer_norm on bf16 (md2fast.py:43-44, eps 1e-5) == bf16((x - mean) / sqrt(var + eps) * g + b) in fp64;
    small-variance rows make the eps term visible (eps 1e-6 would fail)."""
    x = (torch.randn(64, 1152, generator=gen(1)) * 3e-3).to(BF)
    g = (1 + 0.1 * torch.randn(1152, generator=gen(2))).to(BF)
    b = (0.1 * torch.randn(1152, generator=gen(3))).to(BF)
    xd = x.double()
    y = ((xd - xd.mean(1, keepdim=True)) / torch.sqrt(xd.var(1, unbiased=False, keepdim=True) + 1e-5)) * g.double() + b.double()
    out = ov.ln(x, g, b).double()
    assert (out - bfr(y)).abs().max() <= 2 ** -7 * y.abs().max()
    wrong = ((xd - xd.mean(1, keepdim=True)) / torch.sqrt(xd.var(1, unbiased=False, keepdim=True) + 1e-6)) * g.double() + b.double()
    assert (out - bfr(wrong)).abs().max() > 0.05


def test_gelu_tanh_closed_form():
    """gelu = 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))) (tgemm.py:21-25, i8gemm.hip:11), not the erf form."""
    x = torch.linspace(-6, 6, 4001).to(BF)
    xd = x.double()
    ref = 0.5 * xd * (1 + torch.tanh(0.7978845608028654 * (xd + 0.044715 * xd ** 3)))
    assert (ov.gelu(x).double() - bfr(ref)).abs().max() <= 2 ** -8 * 4
    erf = 0.5 * xd * (1 + torch.erf(xd / math.sqrt(2)))
    assert (ov.gelu(x).double() - bfr(erf)).abs().max() > 1e-3  # the two forms are distinguishable here


def test_sdpa_default_scale_and_softmax_brute_force():
    """The oracle's SDPA (default scale D^-0.5, md2fast.py:155; hattn.py:24) vs an fp64 loop over keys."""
    H, T, D = 2, 9, 72
    q, k, v = (torch.randn(1, H, T, D, generator=gen(i)).to(BF) for i in range(3))
    out = F.scaled_dot_product_attention(q, k, v).double()
    ref = torch.zeros(1, H, T, D, dtype=torch.float64)
    for h in range(H):
        for i in range(T):
            s = [sum(q[0, h, i, d].item() * k[0, h, j, d].item() for d in range(D)) / math.sqrt(D) for j in range(T)]
            m = max(s)
            p = [math.exp(x - m) for x in s]
            z = sum(p)
            for j in range(T):
                ref[0, h, i] += p[j] / z * v[0, h, j].double()
    assert (out - ref).abs().max() < 2e-2
    wrong = F.scaled_dot_product_attention(q, k, v, scale=0.125).double()  # a 1/8 scale (TRecViT's) would show
    assert (wrong - ref).abs().max() > 2e-2


# ---------------------------------------------------------------------------------------------- vision
def test_patchify_order_and_normalisation():
    """(u8 / 255 - 0.5) / 0.5 in bf16 steps, patch rows in (c, ky, kx) order (md2fast.py:148-149)."""
    img = torch.randint(0, 256, (1, 378, 378, 3), generator=gen(4), dtype=torch.uint8)
    p = ov.normalize_patchify(img)
    for (gy, gx, c, ky, kx) in [(0, 0, 0, 0, 0), (3, 20, 2, 13, 5), (26, 26, 1, 7, 13), (5, 9, 0, 13, 0)]:
        u = img[0, gy * 14 + ky, gx * 14 + kx, c].item()
        a = torch.tensor(float(u)).to(BF).div(255.0).to(BF)
        expect = ((a.float() - 0.5).to(BF).float() / 0.5).to(BF)
        assert p[0, gy * 27 + gx, c * 196 + ky * 14 + kx] == expect


def _tiny_vision(D=32, Fh=48, H=4):
    w = {}
    g = gen(5)
    for name, shape in (("attn.qkv", (3 * D, D)), ("attn.proj", (D, D)), ("mlp.fc1", (Fh, D)), ("mlp.fc2", (D, Fh))):
        w["blocks.0." + name + ".weight"] = (torch.randn(*shape, generator=g) * 0.2).to(BF)
        w["blocks.0." + name + ".bias"] = (torch.randn(shape[0], generator=g) * 0.2).to(BF)
    for n in ("ln1", "ln2"):
        w[f"blocks.0.{n}.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
        w[f"blocks.0.{n}.bias"] = (0.1 * torch.randn(D, generator=g)).to(BF)
    return w


def test_vision_block_structure_vs_fp64():
    """pre-LN block: x + proj(attn(LN1 x)), then + fc2(gelu(fc1(LN2 .))) (md2fast.py:153-157), fp64 restatement."""
    D, H = 32, 4
    w = _tiny_vision(D, 48, H)
    x = torch.randn(2, 11, D, generator=gen(6)).to(BF)
    out = ov.block(w, 0, x, H=H).double()
    wd = {k: v.double() for k, v in w.items()}
    p = "blocks.0."
    xd = x.double()
    lnd = lambda t, n: F.layer_norm(t, (D,), wd[p + n + ".weight"], wd[p + n + ".bias"], 1e-5)
    qkv = F.linear(lnd(xd, "ln1"), wd[p + "attn.qkv.weight"], wd[p + "attn.qkv.bias"])
    q, k, v = [t.view(2, 11, H, -1).transpose(1, 2) for t in qkv.chunk(3, -1)]
    a = torch.softmax(q @ k.transpose(-1, -2) / math.sqrt(D // H), -1) @ v
    x1 = xd + F.linear(a.transpose(1, 2).reshape(2, 11, D), wd[p + "attn.proj.weight"], wd[p + "attn.proj.bias"])
    hdn = F.linear(lnd(x1, "ln2"), wd[p + "mlp.fc1.weight"], wd[p + "mlp.fc1.bias"])
    hdn = 0.5 * hdn * (1 + torch.tanh(0.7978845608028654 * (hdn + 0.044715 * hdn ** 3)))
    ref = x1 + F.linear(hdn, wd[p + "mlp.fc2.weight"], wd[p + "mlp.fc2.bias"])
    assert ((out - ref).norm() / ref.norm()) < 1e-2
    no_res = ref - x1  # a block missing its second residual is far off
    assert ((out - no_res).norm() / ref.norm()) > 0.3


class _EpilogueLinear(ov.TorchLinear):
    """HLin-protocol Linear that takes GELU and the residual into its epilogue (the same bf16 roundings as torch's
    separate ops) and records which epilogue each call asked for."""
    fused_gelu = True
    fused_res = True
    calls = []

    def __call__(self, x, gelu=False, res=None):
        _EpilogueLinear.calls.append((self.weight.shape, gelu, res is not None))
        y = F.linear(x, self.weight, self.bias)
        y = ov.gelu(y) if gelu else y
        return y if res is None else y + res


def test_tower_with_injected_operators():
    """tower_with (the operator-injected tower the reference-side binding is tested through) with torch's operators
    is the oracle's tower bit for bit; with a Linear advertising fused_gelu / fused_res, fc1 gets gelu=True every
    time, proj and fc2 get the residual only with fuse_res on (USE_FUSED_RES, md2fast.py:51-67), qkv and the patch
    embedding never get either, and the result is unchanged."""
    w = S.vision_weights(0, layers=2)
    img = S.images_u8(1, 1)
    ref = ov.tower(w, img)[0]
    assert torch.equal(ov.tower_with(w, img[0], ov.TorchLinear, ov.TorchAttention), ref)
    for fuse in (False, True):
        _EpilogueLinear.calls = []
        out = ov.tower_with(w, img[0], _EpilogueLinear, ov.TorchAttention, fuse_res=fuse)
        assert torch.equal(out, ref)
        by_shape = {}
        for shape, g, r in _EpilogueLinear.calls:
            by_shape.setdefault(tuple(shape), set()).add((g, r))
        assert by_shape[(4304, 1152)] == {(True, False)}                      # fc1
        assert by_shape[(1152, 4304)] == {(False, fuse)}                      # fc2
        assert by_shape[(3456, 1152)] == {(False, False)}                     # qkv
        assert by_shape[(1152, 1152)] == {(False, fuse)}                      # proj
        assert by_shape[(1152, 588)] == {(False, False)}                      # patch embedding (+ pos, separate)
        assert len(_EpilogueLinear.calls) == 1 + 4 * 2


# ---------------------------------------------------------------------------------------------- text
def test_rope_against_explicit_rotation():
    """rope (md2fast.py:162-167 / fused.py:53-58): a = x[0:16], b = x[16:32] (halves), output pairs interleaved
    (a c - b s, a s + b c), dims 32..63 passed through."""
    x = torch.randn(1, 2, 5, 64, generator=gen(7)).to(BF)
    fr = S.freqs_cis(32, 64)
    pos = torch.arange(10, 15)
    out = ot.rope(x, fr[pos, :, 0], fr[pos, :, 1])
    for h in range(2):
        for t in range(5):
            for j in range(16):
                c, s = fr[pos[t], j, 0].item(), fr[pos[t], j, 1].item()
                a, b = x[0, h, t, j].item(), x[0, h, t, 16 + j].item()
                assert out[0, h, t, 2 * j].item() == pytest.approx(torch.tensor(a * c - b * s).to(BF).item(), abs=2e-2)
                assert out[0, h, t, 2 * j + 1].item() == pytest.approx(torch.tensor(a * s + b * c).to(BF).item(), abs=2e-2)
            assert torch.equal(out[0, h, t, 32:], x[0, h, t, 32:])


def test_freqs_cis_closed_form():
    fr = S.freqs_cis(32, 2048, 10000.0)
    for p, i in [(0, 0), (1, 0), (730, 3), (2047, 15)]:
        ang = p * 10000.0 ** (-2 * i / 32)
        assert fr[p, i, 0].item() == pytest.approx(math.cos(ang), abs=2e-4)
        assert fr[p, i, 1].item() == pytest.approx(math.sin(ang), abs=2e-4)


def _tiny_text(D=64, Fh=96, V=97, L=2):
    g = gen(8)
    w = {"wte": (torch.randn(V, D, generator=g) * 0.5).to(BF)}
    for i in range(L):
        p = f"blocks.{i}."
        w[p + "ln.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
        w[p + "ln.bias"] = (0.1 * torch.randn(D, generator=g)).to(BF)
        for name, shape in (("attn.qkv", (3 * D, D)), ("attn.proj", (D, D)), ("mlp.fc1", (Fh, D)), ("mlp.fc2", (D, Fh))):
            w[p + name + ".weight"] = (torch.randn(*shape, generator=g) * 0.15).to(BF)
            w[p + name + ".bias"] = (torch.randn(shape[0], generator=g) * 0.1).to(BF)
    w["post_ln.weight"], w["post_ln.bias"] = torch.ones(D, dtype=BF), torch.zeros(D, dtype=BF)
    w["lm_head.weight"] = (torch.randn(V, D, generator=g) * 0.3).to(BF)
    w["lm_head.bias"] = torch.zeros(V, dtype=BF)
    return w


def _fp64_text_prefill(w, img, prompt, H, fr, bos):
    """fp64 restatement: prefix non-causal, prompt sees prefix + causal prompt, parallel residual."""
    wd = {k: v.double() for k, v in w.items()}
    D = wd["wte"].shape[1]
    hd = D // H
    x = torch.cat([wd["wte"][bos:bos + 1], img.double(), wd["wte"][prompt]], 0)
    n = x.shape[0]
    P = 1 + img.shape[0]
    mask = torch.zeros(n, n, dtype=torch.bool)
    mask[:, :P] = True
    for i in range(P, n):
        mask[i, P:i + 1] = True
    mask[:P, P:] = False
    cos, sin = fr[:n, :, 0].double(), fr[:n, :, 1].double()

    def rope(t):  # (H, n, hd)
        a, b = t[..., :16], t[..., 16:32]
        o = torch.stack((a * cos - b * sin, a * sin + b * cos), -1).flatten(-2)
        return torch.cat([o, t[..., 32:]], -1)
    i = 0
    while f"blocks.{i}.ln.weight" in wd:
        p = f"blocks.{i}."
        h = F.layer_norm(x, (D,), wd[p + "ln.weight"], wd[p + "ln.bias"], 1e-5)
        q, k, v = F.linear(h, wd[p + "attn.qkv.weight"], wd[p + "attn.qkv.bias"]).split(D, -1)
        q, k, v = (t.view(n, H, hd).transpose(0, 1) for t in (q, k, v))
        q, k = rope(q), rope(k)
        s = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
        a = torch.softmax(s.masked_fill(~mask, float("-inf")), -1) @ v
        a = a.transpose(0, 1).reshape(n, D)
        f1 = F.linear(h, wd[p + "mlp.fc1.weight"], wd[p + "mlp.fc1.bias"])
        f1 = 0.5 * f1 * (1 + torch.tanh(0.7978845608028654 * (f1 + 0.044715 * f1 ** 3)))
        x = F.linear(f1, wd[p + "mlp.fc2.weight"], wd[p + "mlp.fc2.bias"]) + F.linear(a, wd[p + "attn.proj.weight"], wd[p + "attn.proj.bias"]) + x
        i += 1
    h = F.layer_norm(x[-1], (D,), wd["post_ln.weight"], wd["post_ln.bias"], 1e-5)
    return F.linear(h, wd["lm_head.weight"], wd["lm_head.bias"])


def test_text_prefill_vs_fp64():
    """Prefix prefill (mask-free) + prompt prefill (prefix + causal mask, md2fast.py:132-136) + parallel residual +
    post-LN + lm head, against an fp64 restatement that builds the whole mask explicitly."""
    D, H, V = 64, 2, 97
    w = _tiny_text(D, 96, V)
    fr = S.freqs_cis(32, 256)
    img = (torch.randn(13, D, generator=gen(9)) * 0.5).to(BF)
    prompt = torch.randint(0, V, (6,), generator=gen(10))
    m = ot.Text(w, 64, fr, bos=3, H=H)
    lg = m.prefill(img, prompt).double()
    ref = _fp64_text_prefill(w, img, prompt, H, fr, 3)
    assert ((lg - ref).norm() / ref.norm()) < 2e-2


def test_text_decode_step_equals_longer_prefill():
    """A greedy step at position p over the KV cache == the fp64 prefill of the prompt extended by that token
    (decode attends to every cached key; no mask needed for the last query)."""
    D, H, V = 64, 2, 97
    w = _tiny_text(D, 96, V)
    fr = S.freqs_cis(32, 256)
    img = (torch.randn(13, D, generator=gen(11)) * 0.5).to(BF)
    prompt = torch.randint(0, V, (6,), generator=gen(12))
    m = ot.Text(w, 64, fr, bos=3, H=H)
    toks, lgs = m.generate(img, prompt, 3)
    ref = _fp64_text_prefill(w, img, torch.cat([prompt, torch.tensor(toks[:2])]), H, fr, 3)
    assert ((lgs[2].double() - ref).norm() / ref.norm()) < 2e-2
    assert toks[0] == int(torch.argmax(lgs[0]))


def test_query_padded_rows_equal_unpadded_prefill_fp64():
    """The yes/no query (md2fast.py:208-212, 233-238): each question zero-padded to L, its last real row through the
    post-LN and the yes / no rows of the LM head == the fp64 prefill of the unpadded question, restricted to those
    rows. Reading a padded row, a wrong row order or a dropped prefix key would fail it."""
    D, H, V, L = 64, 2, 97, 9
    w = _tiny_text(D, 96, V)
    fr = S.freqs_cis(32, 256)
    img = (torch.randn(13, D, generator=gen(21)) * 0.5).to(BF)
    qs = [torch.randint(0, V, (n,), generator=gen(22 + n)).tolist() for n in (4, 9, 1)]
    yn = [5, 17, 40, 2]
    m = ot.Text(w, 64, fr, bos=3, H=H)
    m.encode(img)
    lg = m.query(qs, L, yn).double()
    full = m.query(qs, L).double()
    for b, q in enumerate(qs):
        ref = _fp64_text_prefill(w, img, torch.tensor(q), H, fr, 3)
        assert ((lg[b] - ref[yn]).norm() / ref[yn].norm()) < 2e-2, b
        assert ((full[b] - ref).norm() / ref.norm()) < 2e-2, b
        assert torch.equal(full[b][yn], lg[b])  # the small head is the full head's rows


def test_decide_margin_closed_form():
    """decide (md2fast.py:270-279): margin = logsumexp(yes) - logsumexp(no)."""
    lg = torch.tensor([0.0, math.log(3.0), math.log(2.0)])  # yes: e^0 + e^ln3 = 4; no: 2
    pred, m = ot.Text.decide(lg, 2)
    assert pred and abs(m - math.log(2.0)) < 1e-6
    pred, m = ot.Text.decide(torch.tensor([math.log(2.0), 0.0, math.log(3.0)]), 1)  # 2 vs 1 + 3
    assert not pred and abs(m - math.log(0.5)) < 1e-6


def test_argmax_first_index_on_ties():
    """torch.argmax (the greedy rule) returns the first index among equal maxima; the GPU argmax key does too."""
    v = torch.tensor([0.5, 2.0, -1.0, 2.0, 2.0]).to(BF)
    assert int(torch.argmax(v)) == 1


# ---------------------------------------------------------------------------------------------- TRecViT
def test_rmsnorm_rounding_chain():
    """pack8.py:222-229: s = sum_fp32 bf(x^2), ms = bf(s / D), rstd = bf(1 / sqrt(bf(ms + 1e-6))),
    y = bf(bf(x rstd) * bf(scale + 1)) -- restated in numpy fp32 step by step."""
    x = torch.randn(16, 768, generator=gen(13)).to(BF)
    sc = (0.1 * torch.randn(768, generator=gen(14))).to(BF)
    out = otr.rmsnorm(x, sc).float().numpy()
    f = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(BF).float().numpy()
    xf = x.float().numpy()
    s = f(xf * xf).sum(axis=1, dtype=np.float32)
    ms = f(s / np.float32(768))
    rstd = f(np.float32(1) / np.sqrt(f(ms + np.float32(1e-6))))
    sc1 = f(sc.float().numpy() + 1)
    ref = f(f(xf * rstd[:, None]) * sc1[None])
    assert np.abs(out - ref).max() <= 2 ** -7 * np.abs(ref).max()
    # and the plain math (no intermediate roundings) agrees to bf16 precision
    plain = xf / np.sqrt((xf.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * (sc.double().numpy() + 1)
    assert np.abs(out - plain).max() < 0.05


def _ssm_case(T=64, C=128, H=2, seed=15):
    g = gen(seed)
    n = lambda *s, std=1.0: torch.randn(*s, generator=g) * std
    return dict(yg=n(T, C).to(BF), xx=n(T, C).to(BF), hist=[n(T, C).to(BF) for _ in range(3)], h0=n(T, C),
                conv_w=n(4, C, std=0.3).to(BF), conv_b=n(C, std=0.1).to(BF),
                a_param=(torch.rand(C, generator=g) * 3.5 - 3.0).to(BF),
                wx=n(H, 64, 64, std=0.15).to(BF), bx=n(H, 64, std=0.3).to(BF),
                wa=n(H, 64, 64, std=0.15).to(BF), ba=n(H, 64, std=0.3).to(BF))


def _run_ssm(d, first, **over):
    a = dict(d, **over)
    return otr.ssm(a["yg"], a["xx"], a["hist"], a["h0"], a["conv_w"], a["conv_b"], a["a_param"], a["wx"], a["bx"],
                   a["wa"], a["ba"], first)


def test_rglru_layer_is_the_ssm_core_with_identity_conv():
    """rglru (RGLRU.forward, cpuemu.py:33-47) is the SSM core with the conv and the y gate taken out: ssm with conv
    taps (0, 0, 0, 1), a zero conv bias and yg = 1 gives xc = x and z = bf(h), so both restatements agree bit for
    bit, first frame (h0 None: y = gated x, h = its fp32 value) and later frames; a later frame also differs from the
    first-frame rule (h0 is used)."""
    d = _ssm_case()
    T, C = d["xx"].shape
    ident = torch.zeros(4, C, dtype=BF)
    ident[3] = 1.0
    ones = torch.ones(T, C, dtype=BF)
    for first in (True, False):
        z, h = _run_ssm(d, first, conv_w=ident, conv_b=torch.zeros(C, dtype=BF), yg=ones)
        y2, h2 = otr.rglru(d["xx"], None if first else d["h0"], d["wx"], d["bx"], d["wa"], d["ba"], d["a_param"])
        assert torch.equal(h, h2) and torch.equal(z, y2) and torch.equal(y2, h2.to(BF)), first
    y1, h1 = otr.rglru(d["xx"], None, d["wx"], d["bx"], d["wa"], d["ba"], d["a_param"])
    assert (h1 - h2).abs().max() > 0.1


def test_ssm_first_frame_is_gated_input():
    """First frame (cpuemu.py:41-42): zero conv history and h = gated_x = bf(xc * sigmoid(gx)), computed here
    independently (conv = current tap * w_3 + b only)."""
    d = _ssm_case()
    z, h = _run_ssm(d, True)
    xc = bfr(bfr(bfr(d["xx"].double() * bfr(d["conv_w"][3].double()))) + bfr(d["conv_b"].double()))
    gx = bfr(bfr(torch.einsum("thi,hij->thj", xc.view(64, 2, 64), d["wx"].double()).reshape(64, 128)) + bfr(d["bx"].double().reshape(-1)))
    gated = bfr(xc * bfr(torch.sigmoid(gx)))
    assert (h.double() - gated).abs().max() <= 2 ** -8 * gated.abs().max()
    assert torch.equal(z, (h.to(BF).float() * d["yg"].float()).to(BF))


def test_ssm_tap_order():
    """conv_w row 0 multiplies the OLDEST frame (t-3), row 3 the current one (ew8.cc:1194-1200 / pack8.py:258)."""
    d = _ssm_case()
    w = torch.zeros_like(d["conv_w"])
    w[0] = 1.0  # only the oldest tap
    _, h_old = _run_ssm(d, False, conv_w=w, conv_b=torch.zeros_like(d["conv_b"]))
    hist = [torch.zeros_like(t) for t in d["hist"]]
    hist[2] = d["hist"][2]  # keep only x_{t-3}
    _, h_same = _run_ssm(d, False, conv_w=w, conv_b=torch.zeros_like(d["conv_b"]), hist=hist)
    assert torch.equal(h_old, h_same)
    hist2 = [torch.zeros_like(t) for t in d["hist"]]
    hist2[0] = d["hist"][2]  # the same data as x_{t-1} must give something else
    _, h_diff = _run_ssm(d, False, conv_w=w, conv_b=torch.zeros_like(d["conv_b"]), hist=hist2)
    assert not torch.equal(h_old, h_diff)


def test_ssm_decay_to_one_keeps_state():
    """a_param -> -inf: softplus -> 0, a -> 1, sqrt(1 - a^2) -> 0: the state is carried unchanged."""
    d = _ssm_case()
    _, h = _run_ssm(d, False, a_param=torch.full_like(d["a_param"], -60.0))
    assert torch.equal(h, d["h0"])


def test_rglru_fixed_point():
    """Constant input over many frames: h converges to the fixed point h* = mult g / (1 - a) (a < 1), i.e.
    B / (1 - A) of the per-frame affine map h -> A h + B."""
    d = _ssm_case(T=8, C=64, H=1)
    d["a_param"] = torch.full_like(d["a_param"], 0.0)
    d["hist"] = [d["xx"]] * 3  # a constant input sequence
    h = d["h0"]
    for _ in range(400):
        _, h = _run_ssm(d, False, h0=h)
    _, h1 = _run_ssm(d, False, h0=torch.zeros_like(h))            # B = h(0)
    _, h2 = _run_ssm(d, False, h0=torch.ones_like(h))             # A + B = h(1)
    A, B = (h2 - h1).double(), h1.double()
    assert (A < 1).all() and (A > 0).all()
    assert (h.double() - B / (1 - A)).abs().max() < 1e-4


U = 2.0 ** -8  # unit roundoff of bf16 (8 significand bits, round to nearest even)


def rglru_fp64(d, variant=None):
    """One non-first RG-LRU frame (pack8.py:253-279, cpuemu.py:37-45) from its mathematical definition in fp64, and a
    first-order bound on the oracle's deviation from it caused by its bf16 roundings. Returns (h, bound).

        xc   = sum_i x_{t-3+i} w_i + b                   (conv_1d, tap 0 = oldest)
        gx   = xc_h Wx_h + bx,   ga = xc_h Wa_h + ba      (block-diagonal gates, W[h][in][out])
        a    = (1 + e^p)^(-8 sigma(ga))                  (= exp(-8 sigma(ga) softplus(p)))
        h    = a h0 + sqrt(1 - a^2) xc sigma(gx)

    `variant` computes a plausible wrong restatement instead (for the negative checks): "sqrt1ma" uses sqrt(1 - a),
    "xc" drops the input gate (xc instead of xc sigma(gx)), "coef4" uses -4 instead of -8, "decay_h0" uses (1 - a) h0,
    "wT" multiplies by the transposed per-head gate matrices.
    The bound follows each rounding site of the oracle's chain (every bf16 rounding contributes u |value| and is
    carried to h through the derivatives), times 1.25 for the second-order terms."""
    T, C = d["xx"].shape
    H = d["wx"].shape[0]
    dd = lambda t: t.double()
    taps = [dd(d["hist"][2]), dd(d["hist"][1]), dd(d["hist"][0]), dd(d["xx"])]
    w = dd(d["conv_w"])
    prods = [t * w[i][None] for i, t in enumerate(taps)]
    xc = sum(prods) + dd(d["conv_b"])[None]
    e_xc = U * (2 * sum(p.abs() for p in prods) + dd(d["conv_b"]).abs()[None] + xc.abs())

    def gate(W, b):
        W = W.transpose(-1, -2) if variant == "wT" else W
        pre = torch.einsum("thi,hij->thj", xc.view(T, H, 64), dd(W)).reshape(T, C)
        e = torch.einsum("thi,hij->thj", e_xc.view(T, H, 64), dd(W).abs()).reshape(T, C)
        g = pre + dd(b).reshape(-1)[None]
        s = torch.sigmoid(g)
        e_g = e + U * pre.abs() + U * g.abs()
        return s, s * (1 - s) * e_g + U * s
    sx, e_sx = gate(d["wx"], d["bx"])
    sa, e_sa = gate(d["wa"], d["ba"])
    p = dd(d["a_param"])[None]
    sp = torch.log1p(torch.exp(p))
    coef = 4.0 if variant == "coef4" else 8.0
    a = (1 + torch.exp(p)) ** (-coef * sa)
    L = -8.0 * sa * sp
    e_L = 8.0 * (e_sa * sp + sa * U * sp) + U * L.abs()
    e_a = a * e_L + U * a
    g = xc * sx
    e_g = e_xc * sx + xc.abs() * e_sx + U * g.abs()
    om = 1 - a * a
    e_om = a * a * (2 * e_L + U) + U * om
    mult = torch.sqrt(om)
    e_mult = e_om / (2 * mult.clamp_min(1e-300)) + U * mult
    nx = g * mult
    e_nx = e_g * mult + g.abs() * e_mult + U * nx.abs()
    h0 = dd(d["h0"])
    if variant == "sqrt1ma":
        nx = g * torch.sqrt(1 - a)
    elif variant == "xc":
        nx = xc * mult
    h = (1 - a) * h0 + nx if variant == "decay_h0" else a * h0 + nx
    bound = 1.25 * (e_a * h0.abs() + e_nx) + 1e-6 * h.abs() + 1e-30
    return h, bound


def _rglru_generic_case(seed):
    """Non-first frame with every tap and both gate matrices in play; a_param U(-3, 0.5) and gate biases so that
    a spans (0, 1) away from both ends, sigma(gx) spans (0.1, 0.9)."""
    d = _ssm_case(T=64, C=128, H=2, seed=seed)
    g = gen(seed + 100)
    d["ba"] = (torch.rand(2, 64, generator=g) * 3 - 2).to(BF)
    d["bx"] = (torch.rand(2, 64, generator=g) * 4 - 2).to(BF)
    d["h0"] = torch.randn(64, 128, generator=g) * 0.5
    return d


def _rglru_gateless_case(seed):
    """The closed form with the gate matrices zero (sigma(gx) = sigma(bx), sigma(ga) = sigma(ba), known exactly) and
    only the current conv tap: h = a h0 + sqrt(1 - a^2) (x w_3 + b) sigma(bx), a = (1 + e^p)^(-8 sigma(ba))."""
    d = _rglru_generic_case(seed)
    d["wx"] = torch.zeros_like(d["wx"])
    d["wa"] = torch.zeros_like(d["wa"])
    d["conv_w"] = d["conv_w"].clone()
    d["conv_w"][:3] = 0
    return d


@pytest.mark.parametrize("case", ["gateless", "generic"])
def test_rglru_update_vs_fp64_closed_form(case):
    """The oracle's later-frame RG-LRU update against the fp64 closed form h = a h0 + sqrt(1 - a^2) xc sigma(gx),
    a = (1 + e^p)^(-8 sigma(ga)), within the bound its own bf16 roundings allow, element by element; and each
    plausible wrong restatement (sqrt(1 - a), the ungated xc, a -4 coefficient, (1 - a) h0) lies outside that bound
    on a large share of the elements, so the check tells them apart."""
    d = (_rglru_gateless_case if case == "gateless" else _rglru_generic_case)(31)
    _, h = _run_ssm(d, False)
    ref, bound = rglru_fp64(d)
    err = (h.double() - ref).abs()
    assert bool((err <= bound).all()), (err - bound).max().item()
    # the bound is tight, not vacuous: a few bf16 ulps (the generic case carries the conv's rounding through the
    # 64-term gate products as well)
    assert bound.median().item() < (0.05 if case == "gateless" else 0.12) * ref.abs().median().item()
    for variant in ("sqrt1ma", "xc", "coef4", "decay_h0") + (("wT",) if case == "generic" else ()):
        wrong, _ = rglru_fp64(d, variant)
        frac = ((h.double() - wrong).abs() > bound).double().mean().item()
        print(case, variant, f"{frac:.2f} of the elements outside the bound")
        assert frac > 0.3, (variant, frac)


def scan_fp64(A, B, h0):
    """The time scan the GPU kernel runs: inclusive prefix over frames of (a, b) o (a', b') = (a' a, a' b + b')."""
    a, b = A.clone(), B.clone()
    Fr = A.shape[0]
    d = 1
    while d < Fr:
        a_new, b_new = a.clone(), b.clone()
        a_new[d:] = a[d:] * a[:-d]
        b_new[d:] = a[d:] * b[:-d] + b[d:]
        a, b = a_new, b_new
        d *= 2
    return a * h0[None] + b


def test_associative_scan_equals_sequential_fp64():
    g = gen(16)
    Fr, C = 37, 50
    A = torch.rand(Fr, C, generator=g, dtype=torch.float64)
    B = torch.randn(Fr, C, generator=g, dtype=torch.float64)
    h0 = torch.randn(C, generator=g, dtype=torch.float64)
    seq = []
    h = h0
    for t in range(Fr):
        h = A[t] * h + B[t]
        seq.append(h)
    assert torch.allclose(scan_fp64(A, B, h0), torch.stack(seq), rtol=1e-12, atol=1e-12)
    # the other composition order is a different (wrong) recurrence
    a, b = A.clone(), B.clone()
    d = 1
    while d < Fr:
        a_new, b_new = a.clone(), b.clone()
        b_new[d:] = a[:-d] * b[d:] + b[:-d]
        a_new[d:] = a[d:] * a[:-d]
        a, b = a_new, b_new
        d *= 2
    assert not torch.allclose(a * h0[None] + b, torch.stack(seq), rtol=1e-6)


def test_trecvit_block_first_frame_vs_fp64():
    """One TRecViT block, first frame, tiny width (2 heads): the oracle's bf16 chain vs an fp64 restatement of
    step8.py:470-488 (RMSNorm (1 + scale), [y | x] split, tanh GELU gate, RG-LRU first frame h = x sigmoid(gx),
    gated MLP gate/up, LN eps 1e-6, attention scale 1/8, erf GELU ViT MLP, residuals)."""
    D, H, Fh = 128, 2, 96
    g = gen(17)
    n = lambda *s, std=0.1: (torch.randn(*s, generator=g) * std).to(BF)
    rb, mb, vb, sb = "blocks.0.ssm_block.recurrent_block.", "blocks.0.ssm_block.mlp_block.", "blocks.0.vit_block.", "blocks.0.ssm_block."
    w = {sb + "temporal_pre_norm.scale": n(D), sb + "channel_pre_norm.scale": n(D)}
    for name, shape in ((rb + "linear_yx", (2 * D, D)), (rb + "linear_out", (D, D)), (mb + "ffw_up", (2 * Fh, D)),
                        (mb + "ffw_down", (D, Fh)), (vb + "self_attention.out_proj", (D, D)), (vb + "mlp.0", (Fh, D)),
                        (vb + "mlp.3", (D, Fh))):
        w[name + ".weight"], w[name + ".bias"] = n(*shape), n(shape[0])
    w[vb + "self_attention.in_proj_weight"], w[vb + "self_attention.in_proj_bias"] = n(3 * D, D), n(3 * D)
    w[rb + "conv_1d.w"], w[rb + "conv_1d.b"] = n(4, D, std=0.3), n(D)
    w[rb + "rg_lru.a_param"] = n(D, std=1.0)
    for gname in ("input_gate", "a_gate"):
        w[rb + f"rg_lru.{gname}.w"], w[rb + f"rg_lru.{gname}.b"] = n(H, 64, 64, std=0.15), n(H, 64, std=0.3)
    for ln in ("ln_1", "ln_2"):
        w[vb + ln + ".weight"], w[vb + ln + ".bias"] = (1 + n(D)).to(BF), n(D)
    x = torch.randn(40, D, generator=g).to(BF)
    m = otr.Model(w, H=H)
    out = m.block(0, x).double()
    wd = {k: v.double() for k, v in w.items()}
    xd = x.double()
    rms = lambda t, s: t / torch.sqrt((t ** 2).mean(1, keepdim=True) + 1e-6) * (1 + s)
    gt = lambda t: 0.5 * t * (1 + torch.tanh(0.7978845608028654 * (t + 0.044715 * t ** 3)))
    y, xx = F.linear(rms(xd, wd[sb + "temporal_pre_norm.scale"]), wd[rb + "linear_yx.weight"], wd[rb + "linear_yx.bias"]).chunk(2, -1)
    xc = xx * wd[rb + "conv_1d.w"][3] + wd[rb + "conv_1d.b"]
    gx = torch.einsum("thi,hij->thj", xc.view(40, H, 64), wd[rb + "rg_lru.input_gate.w"]).reshape(40, D) + wd[rb + "rg_lru.input_gate.b"].reshape(-1)
    hh = xc * torch.sigmoid(gx)
    res = F.linear(hh * gt(y), wd[rb + "linear_out.weight"], wd[rb + "linear_out.bias"]) + xd
    gate, up = F.linear(rms(res, wd[sb + "channel_pre_norm.scale"]), wd[mb + "ffw_up.weight"], wd[mb + "ffw_up.bias"]).chunk(2, -1)
    x1 = F.linear(gt(gate) * up, wd[mb + "ffw_down.weight"], wd[mb + "ffw_down.bias"]) + res
    lnd = lambda t, nm: F.layer_norm(t, (D,), wd[vb + nm + ".weight"], wd[vb + nm + ".bias"], 1e-6)
    q, k, v = F.linear(lnd(x1, "ln_1"), wd[vb + "self_attention.in_proj_weight"], wd[vb + "self_attention.in_proj_bias"]).view(40, 3, H, 64).permute(1, 2, 0, 3)
    a = (torch.softmax(q @ k.transpose(-1, -2) / 8.0, -1) @ v).transpose(0, 1).reshape(40, D)
    x2 = x1 + F.linear(a, wd[vb + "self_attention.out_proj.weight"], wd[vb + "self_attention.out_proj.bias"])
    m0 = F.linear(lnd(x2, "ln_2"), wd[vb + "mlp.0.weight"], wd[vb + "mlp.0.bias"])
    ref = x2 + F.linear(0.5 * m0 * (1 + torch.erf(m0 / math.sqrt(2))), wd[vb + "mlp.3.weight"], wd[vb + "mlp.3.bias"])
    assert ((out - ref).norm() / ref.norm()) < 1e-2


# ---------------------------------------------------------------------------------------------- synthetic inputs
def test_preprocess_bilinear_closed_forms():
    """step8.py:379-383 (F.interpolate bilinear, align_corners=False, then / 127.5 - 1): a 2x downscale averages
    each 2 x 2 block exactly; the same size is the identity; a linear ramp stays linear inside the frame (source
    coordinate scale (d + 0.5) - 0.5); an upscale clamps the first source coordinate at 0."""
    img = torch.randint(0, 256, (1, 512, 512, 3), generator=gen(41), dtype=torch.uint8)
    out = otr.preprocess(img)
    blk = img.double().view(1, 256, 2, 256, 2, 3).mean(dim=(2, 4))
    assert torch.equal(out.double(), (blk.float() / 127.5 - 1.0).double())
    img = torch.randint(0, 256, (1, 256, 256, 3), generator=gen(42), dtype=torch.uint8)
    assert torch.equal(otr.preprocess(img), img.float() / 127.5 - 1.0)
    W = 480
    ramp = (torch.arange(W) // 2).to(torch.uint8)        # 0, 0, 1, 1, ... : linear within pairs
    img = ramp[None, None, :, None].expand(1, 8, W, 3).contiguous()
    raw = (otr.preprocess(img).double() + 1.0) * 127.5
    for d in (10, 100, 200):
        s = 1.875 * (d + 0.5) - 0.5                      # W / 256 = 1.875
        i0 = int(math.floor(s))
        ref = (1 - (s - i0)) * (i0 // 2) + (s - i0) * ((i0 + 1) // 2)
        assert abs(raw[0, 3, d, 0].item() - ref) < 1e-4
    img = torch.randint(0, 256, (1, 128, 128, 3), generator=gen(43), dtype=torch.uint8)
    up = (otr.preprocess(img).double() + 1.0) * 127.5
    assert abs(up[0, 0, 0, 0].item() - img[0, 0, 0, 0].item()) < 1e-4    # d = 0: s = -0.25 -> 0
    s = 0.5 * 1.5 - 0.5                                                     # d = 1: s = 0.25
    ref = (1 - s) * img[0, 0, 0, 1].item() + s * img[0, 0, 1, 1].item()
    assert abs(up[0, 0, 1, 1].item() - ref) < 1e-3


def test_crop_full_grid_equals_plain_step_and_state_moves():
    """CropModel (crop_study.py:147-185): the full-grid crop equals the plain model step bit for bit (the reference's
    own c256 == base check); after a move, the state of patches that left the crop is zero (h and the 3-frame
    history) and the patches in the crop hold state under their absolute index."""
    w = S.trecvit_weights(0, layers=1)
    frames = torch.randint(0, 256, (3, 64, 64, 3), generator=gen(51), dtype=torch.uint8)
    qf = (torch.rand(4, 2, generator=gen(52))).to(BF)
    base, crop = otr.Model(w), otr.CropModel(w)
    for t in range(2):
        assert torch.equal(crop.step_crop(frames[t], qf, 0, 0, 32), base.step(frames[t], qf))
    crop.reset()
    crop.step_crop(frames[0], qf, 4, 4, 8)
    kept = crop.crop_rows(4, 4, 8)
    h_before = crop.lru[0].clone()
    crop.step_crop(frames[1], qf, 6, 4, 8)     # move down by 2 patch rows
    now = set(crop.crop_rows(6, 4, 8).tolist())
    gone = [r for r in kept.tolist() if r not in now]
    assert len(gone) == 16 and crop.lru[0][gone].abs().max() == 0
    assert crop.lru[0][sorted(now)].abs().max() > 0 and h_before[kept].abs().max() > 0
    for k in range(3):
        assert crop.conv[0][k][gone].abs().max() == 0


def test_soft_argmax_closed_forms():
    """step8.py:356-361: a lone peak reads out its own bin; two bins a, b inside the window weigh as
    sigmoid(0.5 (a - b)) (temperature 0.5); bins beyond +-20 of the argmax are ignored; equal maxima take the first
    index's window; a window clipped at the border averages what is left."""
    n = 256
    lg = np.zeros((1, n), np.float32)
    lg[0, 37] = 80.0
    assert abs(otr.soft_argmax(lg)[0] - 37.0) < 1e-4
    lg = np.full((1, n), -1e4, np.float32)
    lg[0, 100], lg[0, 110] = 3.0, 1.0
    p = 1.0 / (1.0 + math.exp(-0.5 * 2.0))
    assert abs(otr.soft_argmax(lg)[0] - (100 * p + 110 * (1 - p))) < 1e-3
    lg[0, 130] = 2.9   # 30 bins from the argmax: masked out
    assert abs(otr.soft_argmax(lg)[0] - (100 * p + 110 * (1 - p))) < 1e-3
    lg = np.zeros((1, n), np.float32)  # all equal: argmax 0, window [0, 20], uniform
    assert abs(otr.soft_argmax(lg)[0] - 10.0) < 1e-4
    lg[0, 200] = lg[0, 250] = 5.0      # equal maxima: the first one's window [180, 220]
    e = np.exp(np.float32(0.5) * lg[0, 180:221].astype(np.float64))
    assert abs(otr.soft_argmax(lg)[0] - (np.arange(180, 221) * e).sum() / e.sum()) < 1e-3


def test_track_heads_mlp_vs_fp64():
    """The head MLP (Linear -> LayerNorm -> erf GELU, twice, -> Linear) against torch fp64 with F.layer_norm and the
    exact erf GELU; the tanh GELU or a LayerNorm without its affine differ by far more than the bound."""
    w = S.trecvit_weights(0, layers=1)
    x = torch.randn(5, 768, generator=gen(31)).to(BF)
    tr, lg, vis = otr.track_heads(x, w)
    wd = {k: v.double() for k, v in w.items() if "head" in k}

    def mlp(h, name, approx="none"):
        for lin, ln in ((0, 1), (3, 4)):
            h = F.linear(h, wd[f"{name}.{lin}.weight"], wd[f"{name}.{lin}.bias"])
            h = F.layer_norm(h, (h.shape[-1],), wd[f"{name}.{ln}.weight"], wd[f"{name}.{ln}.bias"], 1e-5)
            h = F.gelu(h, approximate=approx)
        return F.linear(h, wd[f"{name}.6.weight"], wd[f"{name}.6.bias"])
    ref = mlp(x.double(), "coordinate_head")
    assert np.abs(lg - ref.numpy()).max() < 2e-5  # fp32 vs fp64: measured 1.4e-6
    assert np.abs(vis - mlp(x.double(), "visible_head")[:, 0].numpy()).max() < 2e-5
    assert np.abs(mlp(x.double(), "coordinate_head", "tanh").numpy() - ref.numpy()).max() > 2e-4  # 6e-4
    n = lg.shape[1] // 2
    assert np.allclose(tr[:, 0], otr.soft_argmax(lg[:, :n]) + 0.5) and np.allclose(tr[:, 1], otr.soft_argmax(lg[:, n:]) + 0.5)


def test_synth_is_seeded_per_tensor():
    """A subset of a model gets exactly the tensors the full model would get (per-name seeds)."""
    a = S.vision_weights(0, layers=1)
    b = S.vision_weights(0, layers=2)
    for k, v in a.items():
        assert torch.equal(v, b[k]), k
    assert not torch.equal(S.vision_weights(1, layers=1)["blocks.0.attn.qkv.weight"], a["blocks.0.attn.qkv.weight"])


# ---------------------------------------------------------------------------------------------- W8A8 text linears
def test_quant_rows_rounds_half_away_from_zero_with_floor():
    """tgemm.py:81-91: s = max(amax, 1e-5) / 127, q = trunc(v + 0.5 sign v). Exact ties (v = +-2.5, +-0.5) go away
    from zero (half-to-even would give 2 / 0), the amax element maps to +-127, an all-zero row keeps the 1e-5 floor."""
    x = torch.tensor([[1.0, 0.0, -1.0, 0.0],
                      [0.0, 0.0, 0.0, 0.0]], dtype=torch.float32)
    # amax = 127/64 makes s = 1/64 exactly, so v = 64 x lands exactly on the ties (all values bf16-exact)
    ties = (torch.tensor([[127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 0.0, -127.0]]) / 64).to(torch.bfloat16)
    q, sc = ot.quant_rows(ties)
    assert sc.item() == 1 / 64
    assert q[0].tolist() == [127, 3, -3, 1, -1, 2, 0, -127]
    v = ties.float() / sc[:, None]
    assert torch.round(v)[0].tolist() == [127, 2, -2, 0, 0, 2, 0, -127]  # half-to-even would differ on the ties
    qz, sz = ot.quant_rows(x[1:].to(torch.bfloat16))
    assert sz.item() == np.float32(1e-5) / np.float32(127.0) and int(qz.abs().max()) == 0
    # dequantisation error within half a step everywhere, on random rows
    xr = torch.randn(16, 256, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    qr, sr = ot.quant_rows(xr)
    err = (qr.float() * sr[:, None] - xr.float()).abs()
    assert bool((err <= sr[:, None] * 0.5 * (1 + 1e-5)).all())
    assert bool((qr.abs().amax(1) == 127).all())


def test_quant_weight_round_half_even_and_scale():
    """hgemm.py:101-106: s = amax / 127 per output row, q = round-half-to-even(w / s) clamped to +-127; a zero row
    keeps the 1e-8 floor."""
    w = torch.tensor([[254.0, 5.0, -5.0, 3.0, 1.0], [0.0, 0.0, 0.0, 0.0, 0.0]]).to(torch.bfloat16)
    q, s = ot.quant_weight(w)
    # row 0: s = 2 -> v = [127, 2.5, -2.5, 1.5, 0.5] -> half-to-even [127, 2, -2, 2, 0]
    assert s[0].item() == 2.0 and q[0].tolist() == [127, 2, -2, 2, 0]
    assert s[1].item() == np.float32(1e-8) / np.float32(127.0) and q[1].abs().max() == 0


def test_i8_linear_matches_fp64_brute_force():
    """i8gemm.hip:181-197: the int32 sum is exact (checked against python integers), then fp32
    ((acc * s_x) * s_w) + b in that order, GELU-tanh on the fp32 value, one bf16 rounding."""
    g = torch.Generator().manual_seed(11)
    q = torch.randint(-127, 128, (3, 40), generator=g, dtype=torch.int8)
    wq = torch.randint(-127, 128, (5, 40), generator=g, dtype=torch.int8)
    sx = torch.rand(3, generator=g) * 0.01 + 1e-3
    sw = torch.rand(5, generator=g) * 0.01 + 1e-3
    b = (torch.randn(5, generator=g) * 0.1).to(torch.bfloat16)
    out = ot.i8_linear(q, sx, wq, sw, b)
    outg = ot.i8_linear(q, sx, wq, sw, b, gelu_tanh=True)
    for m in range(3):
        for n in range(5):
            acc = sum(int(q[m, k]) * int(wq[n, k]) for k in range(40))
            v = np.float32(np.float32(np.float32(acc) * np.float32(sx[m])) * np.float32(sw[n])) + np.float32(b[n].float())
            assert out[m, n].float().item() == torch.tensor(float(v)).to(torch.bfloat16).float().item()
            vd = float(v)
            gd = 0.5 * vd * (1 + math.tanh(0.7978845608028654 * (vd + 0.044715 * vd ** 3)))
            assert abs(outg[m, n].float().item() - gd) <= 2 ** -7 * abs(gd) + 1e-6


def test_w8a8_layer_stays_close_to_bf16():
    """The W8A8 decoder restatement shares everything but the four text Linears with the bf16 one: on a 2-layer model
    its prompt logits sit within the int8 quantisation noise of the bf16 logits (and are not identical)."""
    w = S.text_weights(0, layers=2)
    fr = S.freqs_cis(32, 2048)
    img = S.activations(3, (20, 2048), "img")
    p = S.prompt_ids(4, 6)
    lb = ot.Text(w, 64, fr).prefill(img, p).float()
    lq = ot.Text(w, 64, fr, w8a8=True).prefill(img, p).float()
    r = ((lb - lq).norm() / lb.norm()).item()
    assert 1e-4 < r < 5e-2, r
