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
  * the yes/no query: questions zero-padded to L ids, run under the prefix + causal mask, the post-LN row of each
    question's last real token through the LM head restricted to the yes / no rows (lm_small); decide's margin
    logsumexp(yes) - logsumexp(no) in fp32, pred = margin > 0       md2fast.py:128-143, 208-212, 233-238, 270-279
    (the reference runs the nq questions as one batch with nq cache copies of the prefix; rows of a batch are
    independent, so the restatement runs them one at a time over a single cache)
Greedy decode (ours; not in the reference snapshot): each step feeds argmax(logits) (torch.argmax: first index among
equal maxima) at the next position, attending to every cached key (no mask needed: a single query at the end).
freqs_cis uses theta = 10000 (moondream's value; not present in the snapshot: parity unpinned for theta itself).

W8A8 text linears (Text(..., w8a8=True)), the reference's default text path (bench.py:20 --tlin HI8Lin):
  * quant_weight: per-output-channel scale amax / 127 (amax clamped >= 1e-8), round half to even, clamp +-127
                                                                    hgemm.py:101-106 (HI8Lin.__init__)
  * quant_rows: per-token scale max(amax, 1e-5) / 127, v = x / s, q = trunc(v + 0.5 sign(v)) (half away from zero)
                                                                    tgemm.py:81-91 (_quant_rows), hgemm.py:10-16
  * i8_linear: int32 sum of q . wq, then fp32 ((acc * s_x) * s_w) + bias (bias fp32, hgemm.py:116), GELU-tanh on that
    fp32 value when fused (fused_gelu = True), one bf16 rounding   i8gemm.hip:181-197
  * the layer: LN output quantised once and shared by qkv and fc1 (SHARE_QUANT, md2fast.py:52,174); proj and fc2
    quantise their own inputs; residuals added in bf16 outside the GEMM (fused_res = False: lin_res / mlp,
    md2fast.py:55-67)
The LM head stays a bf16 Linear (md2fast.py:115).
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


def quant_weight(w):
    """hgemm.py:101-106: (N, K) bf16 weight -> int8 (N, K), fp32 per-row scale."""
    wf = w.float()
    s = wf.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    return (wf / s[:, None]).round().clamp(-127, 127).to(torch.int8), s


def quant_rows(x):
    """tgemm.py:81-91: per-row dynamic int8 quantisation of a bf16 (M, K) activation -> (int8 (M, K), fp32 (M,))."""
    xf = x.float()
    s = xf.abs().amax(dim=-1).clamp_min(1e-5) / 127.0
    v = xf / s[:, None]
    q = torch.trunc(v + torch.where(v >= 0, 0.5, -0.5)).to(torch.int32)
    return q.to(torch.int8), s


def _int8_dot(q, wq, kc=1024):
    """Exact int32 q wq^T of int8 values on the CPU's fp32 BLAS: every partial sum over a 1024-wide slice of K is an
    integer below 1024 * 127^2 < 2^24, exact in fp32 in any summation order; the slices are added in int64."""
    K = q.shape[1]
    qf = q.float()
    wf = wq if wq.dtype == torch.float32 else wq.float()
    acc = torch.zeros(q.shape[0], wq.shape[0], dtype=torch.int64)
    for k0 in range(0, K, kc):
        acc += (qf[:, k0:k0 + kc] @ wf[:, k0:k0 + kc].t()).to(torch.int64)
    return acc.to(torch.int32)


def i8_linear(q, sx, wq, sw, bias, gelu_tanh=False, out_dtype=BF):
    """i8gemm.hip:181-197: exact int32 accumulation, fp32 ((acc * s_x) * s_w) + b, optional GELU on the fp32 value,
    one bf16 rounding (none with out_dtype float32: the fp32 arbiter). q (M, K) int8, wq (N, K) int8 (or the same
    values as float32, to skip the conversion)."""
    acc = _int8_dot(q, wq)
    v = acc.float() * sx[:, None]
    v = v * sw[None, :]
    if bias is not None:
        v = v + bias.float()[None, :]
    if gelu_tanh:
        v = gelu(v)
    return v.to(out_dtype)


class Text:
    def __init__(self, w, ctx, freqs, bos=50256, H=32, w8a8=False, dtype=BF):
        """dtype: the activation / cache type. BF is the reference's bf16 path; torch.float32 (with fp32 weights)
        is the same op sequence without bf16 roundings, used as the arbiter of near-tied greedy steps (with w8a8, the
        int8 quantisation stays: the weights quantise to the same int8 values, the activations are quantised from
        fp32 values and the dequantised outputs are not rounded)."""
        self.w = w
        self.H = H
        self.w8a8 = w8a8
        self.dt = dtype
        self.D = w["wte"].shape[1]
        self.hd = self.D // H
        n = 0
        while f"blocks.{n}.ln.weight" in w:
            n += 1
        self.n = n
        self.kc = [torch.zeros(1, H, ctx, self.hd, dtype=dtype) for _ in range(n)]
        self.vc = [torch.zeros(1, H, ctx, self.hd, dtype=dtype) for _ in range(n)]
        self.cos, self.sin = freqs[..., 0].contiguous(), freqs[..., 1].contiguous()
        self.bos = bos
        if w8a8:
            self.q = {f"blocks.{i}.{m}": quant_weight(w[f"blocks.{i}.{m}.weight"])
                      for i in range(n) for m in ("attn.qkv", "attn.proj", "mlp.fc1", "mlp.fc2")}
        self.qf = {}

    def _lin(self, name, x, pre=None, gelu_tanh=False):
        """A text Linear: bf16 F.linear (+ separate GELU), or the W8A8 path (pre = the shared quantised input)."""
        w = self.w
        if not self.w8a8:
            y = F.linear(x, w[name + ".weight"], w[name + ".bias"])
            return gelu(y) if gelu_tanh else y
        shp = x.shape
        q, sx = pre if pre is not None else quant_rows(x.reshape(-1, shp[-1]))
        wq, sw = self.q[name]
        if name not in self.qf:  # the int8 values as float32 once (the exact dot runs on the fp32 BLAS)
            self.qf[name] = wq.float()
        return i8_linear(q, sx, self.qf[name], sw, w[name + ".bias"], gelu_tanh, self.dt).view(*shp[:-1], wq.shape[0])

    def layers(self, x, pos0, mask):
        """md2fast.py:169-199 (fuse=False). x (1, n, D)."""
        w, H, hd = self.w, self.H, self.hd
        n = x.shape[1]
        cos, sin = self.cos[pos0:pos0 + n], self.sin[pos0:pos0 + n]
        for i in range(self.n):
            p = f"blocks.{i}."
            h = ln(x, w[p + "ln.weight"], w[p + "ln.bias"])
            pre = quant_rows(h.reshape(n, -1)) if self.w8a8 else None  # shared by qkv and fc1 (md2fast.py:174)
            qkv = self._lin(p + "attn.qkv", h, pre)
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
            res = self._lin(p + "attn.proj", a) + x
            x = self._lin(p + "mlp.fc2", self._lin(p + "mlp.fc1", h, pre, gelu_tanh=True)) + res
        return x

    def logits(self, x_last):
        w = self.w
        return F.linear(ln(x_last, w["post_ln.weight"], w["post_ln.bias"]), w["lm_head.weight"], w["lm_head.bias"])

    def encode(self, img_emb):
        """md2fast.py:201-206: [BOS] + image tokens, mask-free. Returns the prefix hidden states."""
        w = self.w
        x = torch.cat([w["wte"][self.bos:self.bos + 1], img_emb.to(self.dt)], dim=0)[None]
        self.P = x.shape[1]
        return self.layers(x, 0, None)

    @staticmethod
    def prompt_mask(P, L):
        """md2fast.py:132-136: prompt row i sees every prefix key and prompt keys <= i."""
        m = torch.zeros(L, P + L, dtype=torch.bool)
        m[:, :P] = True
        m[:, P:] = torch.tril(torch.ones(L, L, dtype=torch.bool))
        return m[None, None]

    def query(self, questions, L, yn_ids=None):
        """md2fast.py:208-212 with set_questions (md2fast.py:233-238): each question zero-padded to L ids; returns
        (nq, len(yn_ids)) logits of the yes / no rows, or (nq, V) when yn_ids is None. Needs encode() first."""
        w, P = self.w, self.P
        out = []
        for q in questions:
            ids = torch.zeros(L, dtype=torch.int64)
            ids[:len(q)] = torch.as_tensor(q, dtype=torch.int64)
            x = self.layers(F.embedding(ids[None], w["wte"]), P, self.prompt_mask(P, L))
            h = ln(x[0, len(q) - 1], w["post_ln.weight"], w["post_ln.bias"])
            if yn_ids is None:
                out.append(F.linear(h, w["lm_head.weight"], w["lm_head.bias"]))
            else:
                idx = torch.as_tensor(yn_ids)
                out.append(F.linear(h, w["lm_head.weight"][idx], w["lm_head.bias"][idx]))
        return torch.stack(out)

    @staticmethod
    def decide(logits, n_yes):
        """md2fast.py:270-279 on yes/no-row logits: (pred_yes, margin) with margin = logsumexp(yes) -
        logsumexp(no) in fp32."""
        lg = logits.float()
        m = (torch.logsumexp(lg[:n_yes], 0) - torch.logsumexp(lg[n_yes:], 0)).item()
        return m > 0, m

    def prefill(self, img_emb, prompt_ids, return_hidden=False):
        w = self.w
        hp = self.encode(img_emb)
        P = self.P
        L = prompt_ids.shape[0]
        xp = self.layers(F.embedding(prompt_ids[None], w["wte"]), P, self.prompt_mask(P, L))
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
