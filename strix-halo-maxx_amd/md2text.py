"""moondream2 text decoder on the MI355X kernels: prefix prefill (BOS + image tokens, mask-free), masked prompt
prefill, and batch-1 greedy decode with a contiguous bf16 KV cache.

Follows the reference's FastMD2 text path (moondream/gpu/md2fast.py:162-212): the same layer loop
(LN -> qkv -> rope + KV write -> SDPA -> parallel residual `fc2(gelu(fc1(h))) + (proj(a) + x)`), the same prefix /
prompt split and prompt mask (md2fast.py:132-136), the same `lin_cls` plug-in. The reference never decodes (it reads
yes/no logits off one prefill, md2fast.py:10-11); the greedy loop here is the decode the stock HF path runs,
rebuilt for batch-1 HBM streaming:
  * per layer 3 kernels: LN fused into the [qkv | fc1] GEMV, rope + KV append fused into split-KV attention, and
    the fc2 / proj GEMVs fused with the two residual adds;
  * the LM head GEMV carries the argmax, and the next step's embedding lookup reduces it on the device, so one HIP
    graph replays a whole step with the token and position kept in device memory (no host round trip per token).
"""
import torch

from . import _lib, ops
from ._lib import call, ptr, stream
from .synth import TXT, freqs_cis

BF = torch.bfloat16
BOS = 50256  # moondream2's tokenizer bos_id (the Phi / GPT-2 <|endoftext|> id)


class TextDecoder:
    def __init__(self, weights, lin_cls=ops.MxLin, device="cuda", ctx=1024, attn_splits=4, w8a8=False):
        """w8a8: the four text Linears of every layer run the reference's W8A8 path (its default text linear class,
        HI8Lin, moondream/gpu/bench.py:20) in prefill and decode; the LM head stays bf16 (md2fast.py:115)."""
        c = TXT
        self.dev = torch.device(device)
        self.D, self.H, self.hd, self.eps = c["dim"], c["heads"], c["hd"], c["ln_eps"]
        self.ctx = ctx
        dev = self.dev
        g = lambda n: weights[n].to(dev, BF).contiguous()
        f32 = lambda n: weights[n].to(dev, torch.float32).contiguous()
        self.wte = g("wte")
        self.V = self.wte.shape[0]
        n = 0
        while f"blocks.{n}.ln.weight" in weights:
            n += 1
        self.w8a8 = w8a8
        self.blocks = []
        for i in range(n):
            p = f"blocks.{i}."
            # [Wqkv | Wfc1] stored once, fused: the decode GEMV streams both in one pass; the prefill GEMMs use row
            # slices of the same storage (int8 with per-row scales in the W8A8 form: a row's scale is its own, so the
            # fused quantisation equals quantising qkv and fc1 separately)
            wqf = torch.cat([weights[p + "attn.qkv.weight"], weights[p + "mlp.fc1.weight"]]).to(dev, BF).contiguous()
            bqf = torch.cat([weights[p + "attn.qkv.bias"], weights[p + "mlp.fc1.bias"]]).to(dev, torch.float32).contiguous()
            nq = weights[p + "attn.qkv.weight"].shape[0]
            blk = dict(ln=(g(p + "ln.weight"), g(p + "ln.bias")), bqf=bqf, nq=nq)
            if w8a8:
                wq, sq = ops.MxI8Lin.quantize_weight(wqf)
                del wqf
                blk.update(wqf=wq, sqf=sq, qkv=ops.MxI8Lin.from_quantized(wq[:nq], sq[:nq], bqf[:nq]),
                           fc1=ops.MxI8Lin.from_quantized(wq[nq:], sq[nq:], bqf[nq:]),
                           proj=ops.MxI8Lin(weights[p + "attn.proj.weight"], weights[p + "attn.proj.bias"], BF, dev),
                           fc2=ops.MxI8Lin(weights[p + "mlp.fc2.weight"], weights[p + "mlp.fc2.bias"], BF, dev))
                blk["wp"], blk["swp"] = blk["proj"].wq, blk["proj"].sw
                blk["w2"], blk["sw2"] = blk["fc2"].wq, blk["fc2"].sw
            else:
                blk.update(wqf=wqf, qkv=lin_cls(wqf[:nq], bqf[:nq], BF), fc1=lin_cls(wqf[nq:], bqf[nq:], BF),
                           proj=lin_cls(weights[p + "attn.proj.weight"], weights[p + "attn.proj.bias"], BF),
                           fc2=lin_cls(weights[p + "mlp.fc2.weight"], weights[p + "mlp.fc2.bias"], BF))
                blk["wp"], blk["w2"] = blk["proj"].w, blk["fc2"].w
            blk["bp"], blk["b2"] = f32(p + "attn.proj.bias"), f32(p + "mlp.fc2.bias")
            self.blocks.append(blk)
        self.post_ln = (g("post_ln.weight"), g("post_ln.bias"))
        self.w_lm, self.b_lm = g("lm_head.weight"), f32("lm_head.bias")
        self.cs = freqs_cis(c["rot"], max(ctx, 2048), c["theta"]).to(dev).contiguous()
        self.kc = [torch.zeros(1, self.H, ctx, self.hd, device=dev, dtype=BF) for _ in self.blocks]
        self.vc = [torch.zeros(1, self.H, ctx, self.hd, device=dev, dtype=BF) for _ in self.blocks]
        # ---- decode-step device state
        lib = _lib.load()
        self.S = attn_splits
        self.nparts = lib.mx_lm_argmax_nparts(self.V)
        self.part = torch.zeros(self.nparts, device=dev, dtype=torch.int64)
        self.state = torch.zeros(2, device=dev, dtype=torch.int32)
        self.tokens = torch.zeros(ctx, device=dev, dtype=torch.int32)
        self.xd = [torch.zeros(self.D, device=dev, dtype=BF) for _ in range(2)]
        self.qkv_d = torch.zeros(3 * self.D, device=dev, dtype=BF)
        self.g_d = torch.zeros(c["ff"], device=dev, dtype=BF)
        self.a_d = torch.zeros(self.D, device=dev, dtype=BF)
        self.attn_ws = torch.zeros(self.H * self.S * 66, device=dev, dtype=torch.float32)
        self.attn_cnt = torch.zeros(self.H, device=dev, dtype=torch.int32)
        self.logits = torch.zeros(self.V, device=dev, dtype=BF)
        self.pos_base = 0
        self.graph = None

    # ------------------------------------------------------------------ prefill (md2fast.py:169-212)
    def _text_layers(self, x, pos0, causal_from):
        """x (n, D) bf16 tokens at positions pos0 .. pos0 + n - 1; attends to keys 0 .. pos0 + n - 1 (key j visible
        to query i iff j < causal_from or j <= pos0 + i; causal_from=None: all)."""
        n = x.shape[0]
        H, hd = self.H, self.hd
        Tk = pos0 + n
        for i, b in enumerate(self.blocks):
            h = ops.layernorm(x, *b["ln"], eps=self.eps)
            # W8A8: the LN output is quantised once for qkv and fc1 (SHARE_QUANT, md2fast.py:52, 174)
            pre = b["qkv"].quant(h) if self.w8a8 else None
            qkv = b["qkv"](h, pre=pre)
            q = torch.empty(1, H, n, hd, device=self.dev, dtype=BF)
            call("mx_rope_kv", stream(), qkv.data_ptr(), qkv.stride(0), self.cs.data_ptr(), q.data_ptr(),
                 self.kc[i].data_ptr(), self.vc[i].data_ptr(), 1, n, H, self.ctx, pos0, 1, 0)
            a = ops.sdpa(q, self.kc[i][:, :, :Tk], self.vc[i][:, :, :Tk], qpos0=pos0, causal_from=causal_from)
            r = b["proj"](a.view(n, self.D), res=x)
            x = b["fc2"](b["fc1"](h, gelu=True, pre=pre), res=r)
        return x

    def prefill(self, img_emb, prompt_ids):
        """[BOS] + image tokens (mask-free, md2fast.py:201-206), then the prompt (prefix + causal mask,
        md2fast.py:208-212). Leaves the first generated token's argmax in `part` and returns the prompt's hidden states."""
        n_img = img_emb.shape[0]
        x = torch.cat([self.wte[BOS:BOS + 1], img_emb.to(self.dev, BF)], dim=0)
        self._text_layers(x, 0, None)
        P = n_img + 1
        xp = self.wte[prompt_ids.to(self.dev)]
        xp = self._text_layers(xp, P, P)
        self.pos_base = P + xp.shape[0]
        self.lm_argmax(xp[-1], logits=True)
        return xp

    def lm_argmax(self, x_row, logits=False):
        call("mx_ln_gemv_argmax", stream(), x_row.data_ptr(), self.post_ln[0].data_ptr(), self.post_ln[1].data_ptr(),
             float(self.eps), self.w_lm.data_ptr(), self.w_lm.stride(0), self.b_lm.data_ptr(), self.V, self.D,
             ptr(self.logits) if logits else None, self.part.data_ptr(), self.nparts)

    # ------------------------------------------------------------------ decode
    def start_decode(self):
        """Reset the step counter and feed the prefill's argmax token (becomes tokens[0])."""
        self.state.zero_()
        self._embed()

    def _embed(self):
        call("mx_embed_step", stream(), self.part.data_ptr(), self.nparts, self.wte.data_ptr(), self.D,
             self.state.data_ptr(), self.pos_base, self.tokens.data_ptr(), self.xd[0].data_ptr())

    def decode_step(self, logits=False):
        """One greedy step for the token in xd[0] at position state[1]: appends its K/V, computes the next token's
        argmax and embeds it into xd[0]. Graph-capturable (no host reads)."""
        st = stream()
        lib = _lib.load()
        xi = 0
        for i, b in enumerate(self.blocks):
            x, xn = self.xd[xi], self.xd[xi ^ 1]
            if self.w8a8:
                _lib.check(lib.mx_ln_gemv2_i8(st, x.data_ptr(), b["ln"][0].data_ptr(), b["ln"][1].data_ptr(),
                                              float(self.eps), b["wqf"].data_ptr(), b["wqf"].stride(0),
                                              b["sqf"].data_ptr(), b["bqf"].data_ptr(), b["wqf"].shape[0], self.D,
                                              b["nq"], self.qkv_d.data_ptr(), self.g_d.data_ptr(), 1), "mx_ln_gemv2_i8")
            else:
                _lib.check(lib.mx_ln_gemv2(st, x.data_ptr(), b["ln"][0].data_ptr(), b["ln"][1].data_ptr(),
                                           float(self.eps), b["wqf"].data_ptr(), b["wqf"].stride(0), b["bqf"].data_ptr(),
                                           b["wqf"].shape[0], self.D, b["nq"], self.qkv_d.data_ptr(),
                                           self.g_d.data_ptr(), 1), "mx_ln_gemv2")
            _lib.check(lib.mx_decode_attn(st, self.qkv_d.data_ptr(), self.cs.data_ptr(), self.kc[i].data_ptr(),
                                          self.vc[i].data_ptr(), self.H, self.ctx, self.state.data_ptr(), self.S,
                                          float(self.hd ** -0.5), self.attn_ws.data_ptr(), self.attn_cnt.data_ptr(),
                                          self.a_d.data_ptr()), "mx_decode_attn")
            if self.w8a8:
                _lib.check(lib.mx_gemv_dual_res_i8(st, self.g_d.data_ptr(), b["w2"].data_ptr(), b["sw2"].data_ptr(),
                                                   b["b2"].data_ptr(), b["w2"].shape[1], self.a_d.data_ptr(),
                                                   b["wp"].data_ptr(), b["swp"].data_ptr(), b["bp"].data_ptr(),
                                                   b["wp"].shape[1], x.data_ptr(), xn.data_ptr(), self.D),
                           "mx_gemv_dual_res_i8")
            else:
                _lib.check(lib.mx_gemv_dual_res(st, self.g_d.data_ptr(), b["w2"].data_ptr(), b["b2"].data_ptr(),
                                                b["w2"].shape[1], self.a_d.data_ptr(), b["wp"].data_ptr(),
                                                b["bp"].data_ptr(), b["wp"].shape[1], x.data_ptr(), xn.data_ptr(),
                                                self.D), "mx_gemv_dual_res")
            xi ^= 1
        if xi:
            self.xd[0].copy_(self.xd[1])
        self.lm_argmax(self.xd[0], logits=logits)
        self._embed()

    def capture_step(self):
        """HIP graph of one decode step (the state counter makes each replay the next token)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.decode_step()
        self.graph = g
        return g

    def generate(self, img_emb, prompt_ids, n_tokens, use_graph=True):
        """Prefill + greedy decode; returns the n_tokens generated ids (the first comes from the prompt prefill)."""
        self.prefill(img_emb, prompt_ids)
        self.start_decode()
        if use_graph:
            if self.graph is None:
                self.capture_step()  # recording does not execute the step
            for _ in range(n_tokens - 1):
                self.graph.replay()
        else:
            for _ in range(n_tokens - 1):
                self.decode_step()
        return self.tokens[:n_tokens]
