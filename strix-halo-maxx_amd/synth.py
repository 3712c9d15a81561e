"""Seeded synthetic weights and inputs for the three hot-path workloads (no checkpoints are available offline).

Every tensor is drawn from its own torch.Generator seeded by (base seed, crc32(name)), so any subset of a model
(one block, two layers, ...) gets exactly the tensors the full model would get. Weights and biases ~ N(0, 0.02);
LayerNorm gamma = 1, beta = 0. All tensors are returned on the CPU in bf16 unless
stated; callers move them to the device.
TRecViT RMSNorm scales ~ N(0, 0.1), so the (1 + scale) factor differs from 1 per channel.

Parameter names follow the models the reference loads:
  * moondream2 vision / text (md2fast.py:90-94, :108-112 read model.vision.blocks[i].attn.qkv etc.)
  * TAPNext blocks.{i}.ssm_block.recurrent_block.*, .mlp_block.*, .vit_block.* (tapnext/npu/step8.py:158-186, :203-214)
"""
import zlib

import torch

BF = torch.bfloat16

# ---- moondream2 shapes (md2fast.py:24-29; SigLIP so400m vision encoder, Phi-style text model)
VIS = dict(img=378, patch=14, grid=27, ntok=729, dim=1152, heads=16, hd=72, ff=4304, layers=27, proj_inner=8192,
           proj_out=2048, ln_eps=1e-5)
TXT = dict(dim=2048, heads=32, hd=64, rot=32, ff=8192, layers=24, vocab=51200, ln_eps=1e-5, theta=10000.0, ctx=2048)
# ---- TAPNext-style TRecViT (tapnext/npu/step8.py:470-488; pack8.py:10)
TRV = dict(dim=768, heads=12, hd=64, ff_gated=3072, ff_vit=3072, layers=12, img=256, patch=8, n_img=1024, n_q=256,
           conv_taps=4, rms_eps=1e-6, ln_eps=1e-6, head_hidden=256, head_ln_eps=1e-5, head_radius=20)


def _gen(seed, name):
    return torch.Generator().manual_seed((seed * 1000003 + zlib.crc32(name.encode())) & 0x7FFFFFFFFFFFFFFF)


def normal(seed, name, shape, std=0.02, dtype=BF):
    return (torch.randn(*shape, generator=_gen(seed, name)) * std).to(dtype)


def ones(shape):
    return torch.ones(*shape, dtype=BF)


def zeros(shape, dtype=BF):
    return torch.zeros(*shape, dtype=dtype)


# ------------------------------------------------------------------------------------------------ moondream2 vision
def vision_weights(seed=0, layers=None, proj=False):
    """SigLIP tower: patch embedding (Linear 588 -> 1152, = the 14x14/14 conv), pos_emb, `layers` blocks, post_ln,
    optional projection MLP (2304 -> 8192 -> 2048)."""
    c = VIS
    L = c["layers"] if layers is None else layers
    D, F = c["dim"], c["ff"]
    K = 3 * c["patch"] ** 2
    w = {"patch_emb.weight": normal(seed, "patch_emb.weight", (D, K)), "patch_emb.bias": normal(seed, "patch_emb.bias", (D,)),
         "pos_emb": normal(seed, "pos_emb", (1, c["ntok"], D))}
    for i in range(L):
        p = f"blocks.{i}."
        w[p + "ln1.weight"], w[p + "ln1.bias"] = ones((D,)), zeros((D,))
        w[p + "ln2.weight"], w[p + "ln2.bias"] = ones((D,)), zeros((D,))
        for name, shape in (("attn.qkv", (3 * D, D)), ("attn.proj", (D, D)), ("mlp.fc1", (F, D)), ("mlp.fc2", (D, F))):
            w[p + name + ".weight"] = normal(seed, p + name + ".weight", shape)
            w[p + name + ".bias"] = normal(seed, p + name + ".bias", (shape[0],))
    w["post_ln.weight"], w["post_ln.bias"] = ones((D,)), zeros((D,))
    if proj:
        for name, shape in (("proj_mlp.fc1", (c["proj_inner"], 2 * D)), ("proj_mlp.fc2", (c["proj_out"], c["proj_inner"]))):
            w[name + ".weight"] = normal(seed, name + ".weight", shape)
            w[name + ".bias"] = normal(seed, name + ".bias", (shape[0],))
    return w


def images_u8(seed, batch, size=378):
    """Uniform pixels: u8 values uniform in [0, 255] (i.e. uniform [0, 1] after /255), HWC per image."""
    return torch.randint(0, 256, (batch, size, size, 3), generator=_gen(seed, "pixels"), dtype=torch.uint8)


def activations(seed, shape, name="x"):
    return torch.randn(*shape, generator=_gen(seed, name)).to(BF)


# ------------------------------------------------------------------------------------------------ moondream2 text
def text_weights(seed=0, layers=None, vocab=None):
    c = TXT
    L = c["layers"] if layers is None else layers
    V = c["vocab"] if vocab is None else vocab
    D, F = c["dim"], c["ff"]
    w = {"wte": normal(seed, "wte", (V, D))}
    for i in range(L):
        p = f"blocks.{i}."
        w[p + "ln.weight"], w[p + "ln.bias"] = ones((D,)), zeros((D,))
        for name, shape in (("attn.qkv", (3 * D, D)), ("attn.proj", (D, D)), ("mlp.fc1", (F, D)), ("mlp.fc2", (D, F))):
            w[p + name + ".weight"] = normal(seed, p + name + ".weight", shape)
            w[p + name + ".bias"] = normal(seed, p + name + ".bias", (shape[0],))
    w["post_ln.weight"], w["post_ln.bias"] = ones((D,)), zeros((D,))
    w["lm_head.weight"] = normal(seed, "lm_head.weight", (V, D))
    w["lm_head.bias"] = normal(seed, "lm_head.bias", (V,))
    return w


def freqs_cis(rot=32, ctx=2048, theta=10000.0):
    """(ctx, rot/2, 2) fp32 table of (cos, sin) of pos * theta^(-2i/rot): moondream's precomputed rotary table, with
    theta assumed 10000 (the value is not in the reference snapshot)."""
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.float32)[: rot // 2] / rot))
    ang = torch.outer(torch.arange(ctx, dtype=torch.float32), inv)
    return torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1)


def prompt_ids(seed, n, vocab=51200):
    return torch.randint(0, vocab, (n,), generator=_gen(seed, "prompt"), dtype=torch.long)


# ------------------------------------------------------------------------------------------------ TAPNext TRecViT
def trecvit_weights(seed=0, layers=None):
    c = TRV
    L = c["layers"] if layers is None else layers
    D, H = c["dim"], c["heads"]
    w = {}
    for i in range(L):
        rb = f"blocks.{i}.ssm_block.recurrent_block."
        mb = f"blocks.{i}.ssm_block.mlp_block."
        vb = f"blocks.{i}.vit_block."
        sb = f"blocks.{i}.ssm_block."
        w[sb + "temporal_pre_norm.scale"] = normal(seed, sb + "temporal_pre_norm.scale", (D,), std=0.1)
        w[sb + "channel_pre_norm.scale"] = normal(seed, sb + "channel_pre_norm.scale", (D,), std=0.1)
        for name, shape in ((rb + "linear_yx", (2 * D, D)), (rb + "linear_out", (D, D)),
                            (mb + "ffw_up", (2 * c["ff_gated"], D)), (mb + "ffw_down", (D, c["ff_gated"])),
                            (vb + "self_attention.in_proj", (3 * D, D)), (vb + "self_attention.out_proj", (D, D)),
                            (vb + "mlp.0", (c["ff_vit"], D)), (vb + "mlp.3", (D, c["ff_vit"]))):
            wn = name + "_weight" if name.endswith("in_proj") else name + ".weight"
            bn = name + "_bias" if name.endswith("in_proj") else name + ".bias"
            w[wn] = normal(seed, wn, shape)
            w[bn] = normal(seed, bn, (shape[0],))
        w[rb + "conv_1d.w"] = normal(seed, rb + "conv_1d.w", (c["conv_taps"], D))
        w[rb + "conv_1d.b"] = normal(seed, rb + "conv_1d.b", (D,))
        w[rb + "rg_lru.a_param"] = normal(seed, rb + "rg_lru.a_param", (D,), std=1.0)
        w[rb + "rg_lru.input_gate.w"] = normal(seed, rb + "rg_lru.input_gate.w", (H, D // H, D // H))
        w[rb + "rg_lru.input_gate.b"] = normal(seed, rb + "rg_lru.input_gate.b", (H, D // H))
        w[rb + "rg_lru.a_gate.w"] = normal(seed, rb + "rg_lru.a_gate.w", (H, D // H, D // H))
        w[rb + "rg_lru.a_gate.b"] = normal(seed, rb + "rg_lru.a_gate.b", (H, D // H))
        w[vb + "ln_1.weight"], w[vb + "ln_1.bias"] = ones((D,)), zeros((D,))
        w[vb + "ln_2.weight"], w[vb + "ln_2.bias"] = ones((D,)), zeros((D,))
    w["encoder_norm.weight"], w["encoder_norm.bias"] = ones((D,)), zeros((D,))
    P = c["patch"]
    w["lin_proj.weight"] = normal(seed, "lin_proj.weight", (D, 3, P, P))
    w["lin_proj.bias"] = normal(seed, "lin_proj.bias", (D,))
    g = c["img"] // P
    w["image_pos_emb"] = normal(seed, "image_pos_emb", (1, g * g, D))
    w["query_proj.weight"] = normal(seed, "query_proj.weight", (D, 2))
    w["query_proj.bias"] = normal(seed, "query_proj.bias", (D,))
    # tracking heads, fp32 (nn.Sequential: 0 Linear, 1 LayerNorm, 2 GELU, 3 Linear, 4 LayerNorm, 5 GELU, 6 Linear);
    # the coordinate head reads 2 x 256 bins (one per pixel row / column of the 256 x 256 frame)
    Hh, f32 = c["head_hidden"], torch.float32
    for hn, no in (("coordinate_head", 2 * c["img"]), ("visible_head", 1)):
        for i, shape in ((0, (Hh, D)), (3, (Hh, Hh)), (6, (no, Hh))):
            w[f"{hn}.{i}.weight"] = normal(seed, f"{hn}.{i}.weight", shape, std=0.05, dtype=f32)
            w[f"{hn}.{i}.bias"] = normal(seed, f"{hn}.{i}.bias", (shape[0],), dtype=f32)
        for i in (1, 4):
            w[f"{hn}.{i}.weight"] = 1 + normal(seed, f"{hn}.{i}.weight", (Hh,), std=0.1, dtype=f32)
            w[f"{hn}.{i}.bias"] = normal(seed, f"{hn}.{i}.bias", (Hh,), std=0.1, dtype=f32)
    return w


def frames_u8(seed, n, size=256):
    return torch.randint(0, 256, (n, size, size, 3), generator=_gen(seed, "frames"), dtype=torch.uint8)


def query_points(seed, n, size=256):
    """(n, 3) query points (t, y, x) with coordinates uniform in [0, size)."""
    g = _gen(seed, "queries")
    yx = torch.rand(n, 2, generator=g) * size
    return torch.cat([torch.zeros(n, 1), yx], dim=1)
