"""Oracle: the TAPNext TRecViT block, restated on the CPU with torch's bf16 numerics.

The TAPNext model itself (model.py, weights) is external to the reference snapshot; its block is restated from the
reference's own restatements:
  * block order                     tapnext/npu/step8.py:470-488 (region-by-region check against the torch block)
  * RMSNorm  x * rstd * (1 + scale) tapnext/npu/pack8.py:222-229 (rmsnorm_ref), eps 1e-6
  * LayerNorm (fp32 inside, eps 1e-6) pack8.py:232-238 (layernorm_ref)
  * GELU tanh (ssm y gate, gated MLP) / erf (ViT MLP)   pack8.py:241-250, r6/capture.py:5-8
  * conv_1d + gates + RG-LRU + z    pack8.py:253-279 (ssm_ref), r9/cpuemu.py:33-47 (RGLRU.forward); first frame:
                                    zero conv history and h = gated x (step8.py:232-233, cpuemu.py:41-42)
  * gated MLP gate/up split         r6/capture.py:66-69 (`gate, up = ffw_up(x).chunk(2)`)
  * attention: in_proj -> q, k, v heads -> softmax(q k^T / 8) v -> out_proj   r6/capture.py:78-84, pack8.py:10
  * patch embedding + image_pos_emb, queries appended as rows   step8.py:251-267
  * preprocess: bilinear resize to 256 (F.interpolate, align_corners=False, on fp32 pixel values), / 127.5 - 1,
    fp32 until the bf16 conv input                                step8.py:379-383, :256
The query embedding (external embed_queries) is replaced by a linear map of (y, x) / 256: the same stand-in the GPU
path uses; it is outside the block and not part of the parity claim.

Tracking heads (track_heads): the reference's numpy fp32 restatement of model.heads, step8.py:327-362 (heads_np):
each head Linear -> LayerNorm -> GELU erf -> Linear -> LayerNorm -> GELU erf -> Linear in fp32; the coordinate
head's 2n logits read out per half as the expectation of the bin index under softmax(0.5 * logits) * mask, mask =
|argmax - i| <= 20, renormalised, plus 0.5; the visibility head's output is the visibility logit.
"""
import numpy as np
import torch
import torch.nn.functional as F

BF = torch.bfloat16


def f(v):
    """round to bf16 and back to fp32"""
    return v.to(BF).float()


def preprocess(frames_u8, res=256):
    """step8.py:379-383: (F, H, W, 3) uint8 -> (F, res, res, 3) fp32 in [-1, 1]: channels-last float pixels,
    bilinear resize (align_corners=False), then / 127.5 - 1."""
    t = frames_u8.permute(0, 3, 1, 2).float()
    t = F.interpolate(t, size=(res, res), mode="bilinear", align_corners=False)
    return (t / 127.5 - 1.0).permute(0, 2, 3, 1).contiguous()


def rmsnorm(x, scale, eps=1e-6):
    """pack8.py:222-229 in torch: x bf16 [R, D], scale bf16 [D] (sc1 = bf16(scale + 1))."""
    sc1 = (scale.float() + 1).to(BF).float()
    xf = x.float()
    s = f(xf * xf).sum(dim=1, dtype=torch.float32)
    mean = f(s / x.shape[1])
    rstd = f(1.0 / torch.sqrt(f(mean + eps)))
    return f(f(xf * rstd[:, None]) * sc1[None]).to(BF)


def layernorm(x, w, b, eps=1e-6):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def ssm(yg, xx, hist, h0, conv_w, conv_b, a_param, wx, bx, wa, ba, first):
    """pack8.py:253-279 (ssm_ref) for all 12 heads at once. xx / yg bf16 [T, 768]; hist = [x_{t-1}, x_{t-2}, x_{t-3}];
    h0 fp32 [T, 768]; wx / wa [H, 64 in, 64 out]. Returns (z bf16, h fp32)."""
    T, C = xx.shape
    H = wx.shape[0]
    taps = [hist[2], hist[1], hist[0], xx]  # oldest .. current
    if first:
        taps = [torch.zeros_like(xx)] * 3 + [xx]
    s = sum(f(t.float() * f(conv_w[i].float())[None]) for i, t in enumerate(taps))
    xc = f(f(s) + f(conv_b.float())[None])
    xh = xc.double().view(T, H, 64)
    gx_pre = f(f(torch.einsum("thi,hij->thj", xh, wx.double()).reshape(T, C).float()) + f(bx.float().reshape(-1))[None])
    ga_pre = f(f(torch.einsum("thi,hij->thj", xh, wa.double()).reshape(T, C).float()) + f(ba.float().reshape(-1))[None])
    gate_x = f(torch.sigmoid(gx_pre.double()).float())
    gate_a = f(torch.sigmoid(ga_pre.double()).float())
    sp = f(torch.log1p(torch.exp(a_param.double())).float())
    log_a = f(f(-8.0 * gate_a) * sp[None])
    a = f(torch.exp(log_a.double()).float())
    gated = f(xc * gate_x)
    if first:
        h = gated.clone()
    else:
        e2 = f(torch.exp(f(2.0 * log_a).double()).float())
        mult = f(torch.sqrt(f(1.0 - e2)))
        nx = f(gated * mult)
        h = a * h0 + nx
    z = f(f(h) * yg.float())
    return z.to(BF), h


def rglru(x, h0, wx, bx, wa, ba, a_param):
    """RGLRU.forward(x, h0) -> (y, h) of tapnext/npu/r9/cpuemu.py:33-47 with the exact transcendentals (its "exact"
    variant, :66-72: fp64 sigmoid / exp / sqrt, one bf16 rounding each). x bf16 [T, C] (the layer's input, the conv
    output xc), h0 fp32 [T, C] or None (first frame); wx / wa [H, 64 in, 64 out], bx / ba [H, 64]. The gate products
    accumulate in fp64 and round once to bf16, as in `ssm`. Returns (y bf16 = h rounded, h fp32)."""
    T, C = x.shape
    H = wx.shape[0]
    xd = x.double().view(T, H, 64)

    def gate(w, b):  # BlockDiagonalLinear in bf16, then the sigmoid on the bf16 value, rounded
        pre = f(torch.einsum("thi,hij->thj", xd, w.double()).float()) + f(b.float())[None]
        return f(torch.sigmoid(f(pre).double()).float()).reshape(T, C)

    gate_x, gate_a = gate(wx, bx), gate(wa, ba)
    log_a = f(f(-8.0 * gate_a) * f(torch.log1p(torch.exp(a_param.double())).float())[None])
    gated = f(x.float() * gate_x)
    if h0 is None:
        return gated.to(BF), gated
    a = f(torch.exp(log_a.double()).float())
    om = f(1.0 - f(torch.exp(2.0 * log_a.double()).float()))
    mult = f(torch.sqrt(om.double()).float())
    h = a * h0 + f(gated * mult)
    return h.to(BF), h


class Model:
    def __init__(self, w, H=12):
        self.w = w
        self.H = H
        n = 0
        while f"blocks.{n}.ssm_block.temporal_pre_norm.scale" in w:
            n += 1
        self.n = n
        self.reset()

    def reset(self):
        self.hist = [None] * self.n  # [x_{t-1}, x_{t-2}, x_{t-3}] per block
        self.h = [None] * self.n
        self.t = 0

    def embed(self, frame_u8, qfeat):
        w = self.w
        x = preprocess(frame_u8[None])[0].permute(2, 0, 1)[None]
        x = F.conv2d(x.to(BF), w["lin_proj.weight"], w["lin_proj.bias"], stride=w["lin_proj.weight"].shape[-1])
        x = x[0].flatten(1).transpose(0, 1) + w["image_pos_emb"][0]
        q = F.linear(qfeat.to(BF), w["query_proj.weight"], w["query_proj.bias"])
        return torch.cat([x, q], dim=0)

    def block(self, i, x):
        w = self.w
        rb = f"blocks.{i}.ssm_block.recurrent_block."
        mb = f"blocks.{i}.ssm_block.mlp_block."
        vb = f"blocks.{i}.vit_block."
        sb = f"blocks.{i}.ssm_block."
        T, C = x.shape
        first = self.t == 0
        t0 = rmsnorm(x, w[sb + "temporal_pre_norm.scale"])
        y, xx = F.linear(t0, w[rb + "linear_yx.weight"], w[rb + "linear_yx.bias"]).chunk(2, dim=-1)
        yg = F.gelu(y, approximate="tanh")
        hist = self.hist[i] or [torch.zeros_like(xx)] * 3
        h0 = self.h[i] if self.h[i] is not None else torch.zeros(T, C)
        z, h = ssm(yg, xx, hist, h0, w[rb + "conv_1d.w"], w[rb + "conv_1d.b"], w[rb + "rg_lru.a_param"],
                   w[rb + "rg_lru.input_gate.w"], w[rb + "rg_lru.input_gate.b"], w[rb + "rg_lru.a_gate.w"],
                   w[rb + "rg_lru.a_gate.b"], first)
        self.hist[i] = [xx, hist[0], hist[1]]
        self.h[i] = h
        res = F.linear(z, w[rb + "linear_out.weight"], w[rb + "linear_out.bias"]) + x
        l1 = rmsnorm(res, w[sb + "channel_pre_norm.scale"])
        gate, up = F.linear(l1, w[mb + "ffw_up.weight"], w[mb + "ffw_up.bias"]).chunk(2, dim=-1)
        x1 = F.linear(F.gelu(gate, approximate="tanh") * up, w[mb + "ffw_down.weight"], w[mb + "ffw_down.bias"]) + res
        qkv = F.linear(layernorm(x1, w[vb + "ln_1.weight"], w[vb + "ln_1.bias"]), w[vb + "self_attention.in_proj_weight"],
                       w[vb + "self_attention.in_proj_bias"])
        q, k, v = qkv.view(T, 3, self.H, C // self.H).permute(1, 2, 0, 3)
        a = F.scaled_dot_product_attention(q, k, v).transpose(0, 1).reshape(T, C)
        x2 = x1 + F.linear(a, w[vb + "self_attention.out_proj.weight"], w[vb + "self_attention.out_proj.bias"])
        m = F.gelu(F.linear(layernorm(x2, w[vb + "ln_2.weight"], w[vb + "ln_2.bias"]), w[vb + "mlp.0.weight"], w[vb + "mlp.0.bias"]))
        return x2 + F.linear(m, w[vb + "mlp.3.weight"], w[vb + "mlp.3.bias"])

    def step(self, frame_u8, qfeat, return_blocks=False):
        x = self.embed(frame_u8, qfeat)
        hs = [x]
        for i in range(self.n):
            x = self.block(i, x)
            hs.append(x)
        self.t += 1
        fin = layernorm(x, self.w["encoder_norm.weight"], self.w["encoder_norm.bias"])
        return (fin, hs) if return_blocks else fin


class CropModel(Model):
    """crop_study.py:147-185 (CropTracker, shift=True) on the restated block: per block, the RG-LRU state and the
    3-frame conv history of the image tokens live in buffers indexed by absolute patch (grid x grid rows); a frame
    runs the block on the n x n crop's tokens (their patch embedding + their slice of the position embedding) and the
    queries, with the state rows of those patches (crop_study.py:162-176), then zeroes every patch row and writes
    back the crop's new state (crop_study.py:178-182). The first frame of the video runs without state."""

    def __init__(self, w, H=12, grid=32):
        self.grid = grid
        super().__init__(w, H)

    def reset(self):
        super().reset()
        G2 = self.grid * self.grid
        D = self.w["encoder_norm.weight"].shape[0]
        self.lru = [torch.zeros(G2, D) for _ in range(self.n)]
        self.conv = [[torch.zeros(G2, D, dtype=BF) for _ in range(3)] for _ in range(self.n)]  # x_{t-1..t-3}
        self.qs = [None] * self.n  # the query tokens' (h, history), kept by query slot

    def crop_rows(self, r0, c0, n):
        ar = torch.arange(n)
        return ((r0 + ar)[:, None] * self.grid + (c0 + ar)[None]).flatten()

    def step_crop(self, frame_u8, qfeat, r0, c0, n):
        idx = self.crop_rows(r0, c0, n)
        G2, hw = self.grid * self.grid, n * n
        xf = self.embed(frame_u8, qfeat)       # a patch's embedding depends on its own pixels only
        x = torch.cat([xf[idx], xf[G2:]])
        first = self.t == 0
        for i in range(self.n):
            if first:
                self.hist[i], self.h[i] = None, None
            else:
                qh, qhist = self.qs[i]
                self.h[i] = torch.cat([self.lru[i][idx], qh])
                self.hist[i] = [torch.cat([self.conv[i][k][idx], qhist[k]]) for k in range(3)]
            x = self.block(i, x)
            self.lru[i].zero_()                 # tokens outside the crop lose their state
            for k in range(3):
                self.conv[i][k].zero_()
                self.conv[i][k][idx] = self.hist[i][k][:hw]
            self.lru[i][idx] = self.h[i][:hw]
            self.qs[i] = (self.h[i][hw:], [hk[hw:] for hk in self.hist[i]])
        self.t += 1
        return layernorm(x, self.w["encoder_norm.weight"], self.w["encoder_norm.bias"])


def _head_mlp(x, p):
    """step8.py:347-355: two (Linear, LayerNorm, erf GELU) stages then a Linear, numpy fp32. p: torch-layout
    (out, in) weights w0 / w3 / w6, biases, LayerNorm g1 / b1 / g4 / b4 and eps e1 / e4 (nn.Sequential indices)."""
    erf = lambda a: torch.erf(torch.from_numpy(np.ascontiguousarray(a))).numpy()
    for lin, ln in ((0, 1), (3, 4)):
        h = x @ p[f"w{lin}"].T + p[f"b{lin}"]
        mu = h.mean(-1, keepdims=True)
        var = ((h - mu) ** 2).mean(-1, keepdims=True)
        h = (h - mu) / np.sqrt(var + np.float32(p[f"e{ln}"])) * p[f"g{ln}"] + p[f"b{ln}"]
        x = 0.5 * h * (1.0 + erf(h * np.float32(0.7071067811865476)))
    return x @ p["w6"].T + p["b6"]


def soft_argmax(logits, radius=20):
    """step8.py:356-361 on (Q, n) fp32 logits: E[i] under softmax(0.5 * logits) masked to |argmax - i| <= radius and
    renormalised (argmax: first index among equal maxima)."""
    n = logits.shape[-1]
    idx = np.arange(n, dtype=np.float32)
    am = logits.argmax(-1)[:, None]
    mask = np.abs(am - idx) <= radius
    z = logits * np.float32(0.5)
    e = np.exp(z - z.max(-1, keepdims=True))
    pr = e / e.sum(-1, keepdims=True) * mask
    pr = pr / pr.sum(-1, keepdims=True)
    return (pr * idx).sum(-1)


def head_params(w, name, eps=1e-5):
    """numpy fp32 parameters of one head from the weight dict (nn.Sequential indices 0 / 1 / 3 / 4 / 6)."""
    g = lambda k: w[k].float().numpy()
    p = {}
    for i in (0, 3, 6):
        p[f"w{i}"], p[f"b{i}"] = g(f"{name}.{i}.weight"), g(f"{name}.{i}.bias")
    for i in (1, 4):
        p[f"g{i}"], p[f"b{i}"], p[f"e{i}"] = g(f"{name}.{i}.weight"), g(f"{name}.{i}.bias"), eps
    return p


def track_heads(xq, w, eps=1e-5, radius=20):
    """step8.py:333-362 (heads_np): encoder-normed query rows xq (Q, D) -> tracks (Q, 2) = (half 0, half 1)
    readouts + 0.5, coordinate logits (Q, 2n), visibility logits (Q,). All numpy fp32."""
    x = np.asarray(xq.float().numpy() if torch.is_tensor(xq) else xq, np.float32)
    logits = _head_mlp(x, head_params(w, "coordinate_head", eps))
    n = logits.shape[-1] // 2
    tracks = np.stack([soft_argmax(logits[:, :n], radius), soft_argmax(logits[:, n:], radius)], -1) + np.float32(0.5)
    vis = _head_mlp(x, head_params(w, "visible_head", eps))[:, 0]
    return tracks, logits, vis
