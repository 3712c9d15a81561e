"""Oracle: the moondream2 SigLIP vision tower, restated from the reference's PyTorch bf16 path on the CPU.

Restates moondream/gpu/md2fast.py:
  * Lin = F.linear in bf16                          md2fast.py:33-40
  * _ln = F.layer_norm(eps 1e-5), gelu = tanh GELU  md2fast.py:43-48
  * mlp / lin_res (unfused: bf16 result, then +res) md2fast.py:55-67 (USE_FUSED_RES = False, :51)
  * _vision: normalise, patchify, patch_emb + pos, 27 blocks, post_ln, cat[x,x] projection   md2fast.py:147-160
Everything runs in torch bf16 on the CPU, exactly the op sequence of the reference (F.scaled_dot_product_attention
on (1, H, T, D) transposed views, as md2fast.py:155).
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
