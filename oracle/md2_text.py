"""Oracle: the moondream2 text decoder, restated from the reference's PyTorch bf16 path on the CPU, plus the greedy
decode loop the stock model runs (the reference's fast path stops at the prompt prefill).

Restates moondream/gpu/md2fast.py:
  * _ln / gelu / Lin (F.linear) / mlp / lin_res (unfused)          md2fast.py:33-67
  * _rope: partial rotary on dims 0..31, non-interleaved halves in, interleaved pairs out, fp32 math, bf16 store
                                                                    md2fast.py:162-167 (== fused.py:53-58 ref_rope)
  * _text_layers (fuse=False branch): LN -> qkv -> rope(q), rope(k) -> KV write -> SDPA (mask-free for the prefix,
    masked for the prompt) -> x = mlp(fc1, fc2, h, res=proj(a) + x)  md2fast.py:169-199
  * _encode: x = cat[wte[bos], img_emb]; prefix prefill            md2fast.py:201-206
  * prompt mask: row i sees all prefix keys and prompt keys <= i  md2fast.py:132-136
  * lm head on the post-LN last position                          md2fast.py:208-212
Greedy decode (ours; not in the reference snapshot): each step feeds argmax(logits) (torch.argmax: first index among
equal maxima) at the next position, attending to every cached key (no mask needed: a single query at the end).
freqs_cis uses theta = 10000 (moondream's value; not present in the snapshot: parity unpinned for theta itself).
"""
import torch
import torch.nn.functional as F

BF = torch.bfloat16
ROT = 32


def ln(x, w, b, eps=1e-5):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def gelu(x):
    return F.gelu(x, approximate="tanh")


def rope(x, cos, sin):
    """md2fast.py:162-167: x (B, H, n, 64) bf16; cos/sin (n, 16) fp32."""
    xr, xp = x[..., :ROT], x[..., ROT:]
    a, b = xr[..., :ROT // 2], xr[..., ROT // 2:]
    cos = cos[None, None]
    sin = sin[None, None]
    o = torch.stack((a * cos - b * sin, a * sin + b * cos), dim=-1).flatten(-2)
    return torch.cat([o.to(x.dtype), xp], dim=-1)


class Text:
    def __init__(self, w, ctx, freqs, bos=50256, H=32):
        self.w = w
        self.H = H
        self.D = w["wte"].shape[1]
        self.hd = self.D // H
        n = 0
        while f"blocks.{n}.ln.weight" in w:
            n += 1
        self.n = n
        self.kc = [torch.zeros(1, H, ctx, self.hd, dtype=BF) for _ in range(n)]
        self.vc = [torch.zeros(1, H, ctx, self.hd, dtype=BF) for _ in range(n)]
        self.cos, self.sin = freqs[..., 0].contiguous(), freqs[..., 1].contiguous()
        self.bos = bos

    def layers(self, x, pos0, mask):
        """md2fast.py:169-199 (fuse=False). x (1, n, D)."""
        w, H, hd = self.w, self.H, self.hd
        n = x.shape[1]
        cos, sin = self.cos[pos0:pos0 + n], self.sin[pos0:pos0 + n]
        for i in range(self.n):
            p = f"blocks.{i}."
            h = ln(x, w[p + "ln.weight"], w[p + "ln.bias"])
            qkv = F.linear(h, w[p + "attn.qkv.weight"], w[p + "attn.qkv.bias"])
            q, k, v = qkv.split([H * hd] * 3, dim=-1)
            q = rope(q.view(1, n, H, hd).transpose(1, 2), cos, sin)
            k = rope(k.view(1, n, H, hd).transpose(1, 2), cos, sin)
            v = v.view(1, n, H, hd).transpose(1, 2)
            self.kc[i][:, :, pos0:pos0 + n] = k
            self.vc[i][:, :, pos0:pos0 + n] = v
            if mask is None and pos0 == 0:
                a = F.scaled_dot_product_attention(q, k, v)
            else:
                a = F.scaled_dot_product_attention(q, self.kc[i][:, :, :pos0 + n], self.vc[i][:, :, :pos0 + n], attn_mask=mask)
            a = a.transpose(1, 2).reshape(1, n, H * hd)
            res = F.linear(a, w[p + "attn.proj.weight"], w[p + "attn.proj.bias"]) + x
            x = F.linear(gelu(F.linear(h, w[p + "mlp.fc1.weight"], w[p + "mlp.fc1.bias"])),
                         w[p + "mlp.fc2.weight"], w[p + "mlp.fc2.bias"]) + res
        return x

    def logits(self, x_last):
        w = self.w
        return F.linear(ln(x_last, w["post_ln.weight"], w["post_ln.bias"]), w["lm_head.weight"], w["lm_head.bias"])

    def prefill(self, img_emb, prompt_ids, return_hidden=False):
        w = self.w
        x = torch.cat([w["wte"][self.bos:self.bos + 1], img_emb.to(BF)], dim=0)[None]
        hp = self.layers(x, 0, None)
        P = x.shape[1]
        L = prompt_ids.shape[0]
        m = torch.zeros(L, P + L, dtype=torch.bool)
        m[:, :P] = True
        m[:, P:] = torch.tril(torch.ones(L, L, dtype=torch.bool))
        xp = self.layers(F.embedding(prompt_ids[None], w["wte"]), P, m[None, None])
        self.pos = P + L
        lg = self.logits(xp[0, -1])
        return (lg, hp, xp) if return_hidden else lg

    def step(self, token):
        x = self.w["wte"][token][None, None]
        h = self.layers(x, self.pos, None)
        self.pos += 1
        return self.logits(h[0, -1])

    def generate(self, img_emb, prompt_ids, n_tokens):
        """Greedy: returns (tokens, per-token logits used to pick them)."""
        lg = self.prefill(img_emb, prompt_ids)
        toks, lgs = [], []
        for t in range(n_tokens):
            tok = int(torch.argmax(lg))
            toks.append(tok)
            lgs.append(lg)
            if t + 1 < n_tokens:
                lg = self.step(tok)
        return toks, lgs
