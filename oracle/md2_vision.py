"""Oracle: the moondream2 SigLIP vision tower, restated from the reference's PyTorch bf16 path on the CPU.

Restates moondream/gpu/md2fast.py:
  * Lin = F.linear in bf16                          md2fast.py:33-40
  * _ln = F.layer_norm(eps 1e-5), gelu = tanh GELU  md2fast.py:43-48
  * mlp / lin_res (unfused: bf16 result, then +res) md2fast.py:55-67 (USE_FUSED_RES = False, :51)
  * _vision: normalise, patchify, patch_emb + pos, 27 blocks, post_ln, cat[x,x] projection   md2fast.py:147-160
Everything runs in torch bf16 on the CPU, exactly the op sequence of the reference (F.scaled_dot_product_attention
on (1, H, T, D) transposed views, as md2fast.py:155).

`tower_with` runs the same tower with the Linear and attention operator classes injected (the reference's plug-in
point, FastMD2(model, lin_cls=..., hattn=...), md2fast.py:71, 87-94): a Linear follows hgemm.HLin's protocol
(`cls(weight, bias, dtype)`, `__call__(x, gelu=False, res=None)`, flags `fused_gelu` / `fused_res`,
hgemm.py:139-178) and the attention hattn.Attn's (`cls(H, T, D)`, `__call__(q, k, v)` on (1, H, T, D) views ->
(1, T, H*D), hattn.py:17-37). GELU and residual adds move into a Linear's epilogue exactly when its flags (and, for
the residual, the USE_FUSED_RES switch, md2fast.py:51) say so (md2fast.py:55-67). Test infrastructure: it drives an
operator binding under test through the reference's dataflow; with the default torch operators it is `tower`.
"""
import torch
import torch.nn.functional as F

BF = torch.bfloat16
IMG, PATCH = 378, 14
GRID = IMG // PATCH
NTOK = GRID * GRID


def lin(x, w, b):
    return F.linear(x, w, b)


def ln(x, w, b, eps=1e-5):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def gelu(x):
    return F.gelu(x, approximate="tanh")


def normalize_patchify(img_u8):
    """md2fast.py:148-149 for a batch: (B, 378, 378, 3) u8 -> (B, 729, 588) bf16, per-patch order (c, ky, kx)."""
    B = img_u8.shape[0]
    x = img_u8.permute(0, 3, 1, 2).to(BF).div_(255.0).sub_(0.5).div_(0.5)
    return x.reshape(B, 3, GRID, PATCH, GRID, PATCH).permute(0, 2, 4, 1, 3, 5).reshape(B, NTOK, 3 * PATCH * PATCH)


def block(w, i, x, H=16):
    """One pre-LN block, md2fast.py:153-157. x (B, T, D) bf16."""
    p = f"blocks.{i}."
    B, T, D = x.shape
    h = ln(x, w[p + "ln1.weight"], w[p + "ln1.bias"])
    qkv = lin(h, w[p + "attn.qkv.weight"], w[p + "attn.qkv.bias"])
    q, k, v = [t.view(B, T, H, -1).transpose(1, 2) for t in qkv.chunk(3, dim=-1)]
    a = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(B, T, D)
    x = lin(a, w[p + "attn.proj.weight"], w[p + "attn.proj.bias"]) + x
    h2 = ln(x, w[p + "ln2.weight"], w[p + "ln2.bias"])
    return lin(gelu(lin(h2, w[p + "mlp.fc1.weight"], w[p + "mlp.fc1.bias"])), w[p + "mlp.fc2.weight"], w[p + "mlp.fc2.bias"]) + x


def embed(w, img_u8):
    x = normalize_patchify(img_u8)
    return lin(x, w["patch_emb.weight"], w["patch_emb.bias"]) + w["pos_emb"]


def tower(w, img_u8, layers=None, project=False, return_blocks=False):
    """md2fast.py:147-160 -> (B, 729, 1152) post-LN features [or (B, 729, 2048) projected]."""
    x = embed(w, img_u8)
    n = 0
    while f"blocks.{n}.ln1.weight" in w:
        n += 1
    n = n if layers is None else min(n, layers)
    hs = [x]
    for i in range(n):
        x = block(w, i, x)
        hs.append(x)
    x = ln(x, w["post_ln.weight"], w["post_ln.bias"])
    if project:
        feats = torch.cat([x, x], dim=-1)
        x = lin(gelu(lin(feats, w["proj_mlp.fc1.weight"], w["proj_mlp.fc1.bias"])), w["proj_mlp.fc2.weight"], w["proj_mlp.fc2.bias"])
    return (x, hs) if return_blocks else x


class TorchLinear:
    """F.linear in bf16 with the HLin protocol and no fused epilogues (what the oracle's `lin` computes)."""
    fused_gelu = False
    fused_res = False

    def __init__(self, weight, bias, dtype):
        self.weight, self.bias = weight.to(dtype), None if bias is None else bias.to(dtype)

    def __call__(self, x, gelu=False, res=None):
        if gelu or res is not None:
            raise ValueError("TorchLinear has no fused epilogue")
        return F.linear(x, self.weight, self.bias)


class TorchAttention:
    """F.scaled_dot_product_attention with hattn.Attn's protocol: (1, H, T, D) views -> (1, T, H*D)."""

    def __init__(self, H, T, D):
        self.H, self.D = H, D

    def __call__(self, q, k, v):
        B, H, T, D = q.shape
        return F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(B, T, H * D)


def _run_linear(layer, x, act=False, res=None, fuse_res=False):
    """One Linear of the block with an optional tanh GELU after it and an optional residual add after that. Each of
    the two goes into the layer's epilogue when the layer advertises it (fused_gelu; fused_res with the fuse_res
    switch on), as md2fast.mlp / lin_res decide (md2fast.py:55-67); otherwise it is torch's separate bf16 op on the
    layer's bf16 output."""
    epi = {}
    if act and getattr(layer, "fused_gelu", False):
        epi["gelu"], act = True, False
    if res is not None and fuse_res and getattr(layer, "fused_res", False):
        epi["res"], res = res, None
    y = layer(x, **epi)
    if act:
        y = gelu(y)
    return y if res is None else y + res


def tower_with(w, img_u8, linear_cls, attention_cls, device="cpu", fuse_res=False, H=16):
    """md2fast.py:147-160 (batch of one crop) with injected operator classes; returns (729, 1152) post-LN features.
    Weights are moved to `device` and wrapped once per Linear, as FastMD2's constructor does (md2fast.py:87-94)."""
    dev = torch.device(device)
    wt = lambda n: w[n].to(dev)
    make = lambda n: linear_cls(wt(n + ".weight"), wt(n + ".bias"), BF)
    n_blocks = 0
    while f"blocks.{n_blocks}.ln1.weight" in w:
        n_blocks += 1
    layers = []
    for i in range(n_blocks):
        p = f"blocks.{i}."
        layers.append({k: make(p + name) for k, name in
                       (("qkv", "attn.qkv"), ("proj", "attn.proj"), ("fc1", "mlp.fc1"), ("fc2", "mlp.fc2"))})
        for k in ("ln1", "ln2"):
            layers[-1][k] = (wt(p + k + ".weight"), wt(p + k + ".bias"))
    attend = attention_cls(H, NTOK, 1152 // H)
    x = _run_linear(make("patch_emb"), normalize_patchify(img_u8[None].to(dev)), res=wt("pos_emb"), fuse_res=False)
    for L in layers:
        heads = [t.view(1, NTOK, H, -1).transpose(1, 2) for t in _run_linear(L["qkv"], ln(x, *L["ln1"])).chunk(3, -1)]
        x = _run_linear(L["proj"], attend(*heads), res=x, fuse_res=fuse_res)
        x = _run_linear(L["fc2"], _run_linear(L["fc1"], ln(x, *L["ln2"]), act=True), res=x, fuse_res=fuse_res)
    return ln(x, wt("post_ln.weight"), wt("post_ln.bias"))[0]
