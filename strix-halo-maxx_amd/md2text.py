"""moondream2 text decoder on the MI355X kernels: prefix prefill (BOS + image tokens, mask-free), masked prompt
prefill, the batched yes/no query, and batch-1 greedy decode with a contiguous bf16 KV cache.

Follows the reference's FastMD2 text path (moondream/gpu/md2fast.py:162-212): the same layer loop
(LN -> qkv -> rope + KV write -> SDPA -> parallel residual `fc2(gelu(fc1(h))) + (proj(a) + x)`), the same prefix /
prompt split and prompt mask (md2fast.py:132-136), the same `lin_cls` plug-in. The reference never decodes (it reads
yes/no logits off one prefill, md2fast.py:10-11); the greedy loop here is the decode the stock HF path runs,
rebuilt for batch-1 HBM streaming:
  * per layer 3 kernels: LN fused into the [qkv | fc1] GEMV, rope + KV append fused into split-KV attention, and
    the fc2 / proj GEMVs fused with the two residual adds;
  * the LM head GEMV carries the argmax, and the next step's embedding lookup reduces it on the device, so one HIP
    graph replays a whole step with the token and position kept in device memory (no host round trip per token).
The yes/no query is the reference's own fast path (FastMD2._encode / _query / decide, md2fast.py:201-212, 266-279):
nq questions share the image prefix, whose K/V the prefix prefill writes into every question's cache slot; the
questions, zero-padded to L tokens, run as one batch of nq * L rows under the prefix + causal mask; the last real
token of each question goes through the final LN and the LM head restricted to the yes / no token rows.
"""
import warnings

import torch

from . import _lib, ops
from ._lib import call, ptr, stream
from .synth import TXT, freqs_cis

BF = torch.bfloat16
BOS = 50256  # moondream2's tokenizer bos_id (the Phi / GPT-2 <|endoftext|> id)


class TextDecoder:
    def __init__(self, weights, lin_cls=ops.MxLin, device="cuda", ctx=1024, attn_splits=1, w8a8=False, nq=1, L=32,
                 yes_ids=(), no_ids=()):
        """w8a8: the four text Linears of every layer run the reference's W8A8 path (its default text linear class,
        HI8Lin, moondream/gpu/bench.py:20) in prefill and decode; the LM head stays bf16 (md2fast.py:115).
        nq, L: questions per query and tokens per question (the reference's NQ, L, md2fast.py:71-86); the KV cache
        holds nq slots (decode uses slot 0). yes_ids / no_ids: the token ids the yes/no head keeps (the reference
        derives them from its tokenizer, md2fast.py:138-142; there is no tokenizer here, the caller passes them)."""
        c = TXT
        self.dev = torch.device(device)
        self.D, self.H, self.hd, self.eps = c["dim"], c["heads"], c["hd"], c["ln_eps"]
        self.ctx = ctx
        self.nq, self.L = nq, L
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
            nqkv = weights[p + "attn.qkv.weight"].shape[0]
            blk = dict(ln=(g(p + "ln.weight"), g(p + "ln.bias")), bqf=bqf, nq=nqkv)
            if w8a8:
                wq, sq = ops.MxI8Lin.quantize_weight(wqf)
                del wqf
                blk.update(wqf=wq, sqf=sq, qkv=ops.MxI8Lin.from_quantized(wq[:nqkv], sq[:nqkv], bqf[:nqkv]),
                           fc1=ops.MxI8Lin.from_quantized(wq[nqkv:], sq[nqkv:], bqf[nqkv:]),
                           proj=ops.MxI8Lin(weights[p + "attn.proj.weight"], weights[p + "attn.proj.bias"], BF, dev),
                           fc2=ops.MxI8Lin(weights[p + "mlp.fc2.weight"], weights[p + "mlp.fc2.bias"], BF, dev))
                blk["wp"], blk["swp"] = blk["proj"].wq, blk["proj"].sw
                blk["w2"], blk["sw2"] = blk["fc2"].wq, blk["fc2"].sw
            else:
                blk.update(wqf=wqf, qkv=lin_cls(wqf[:nqkv], bqf[:nqkv], BF), fc1=lin_cls(wqf[nqkv:], bqf[nqkv:], BF),
                           proj=lin_cls(weights[p + "attn.proj.weight"], weights[p + "attn.proj.bias"], BF),
                           fc2=lin_cls(weights[p + "mlp.fc2.weight"], weights[p + "mlp.fc2.bias"], BF))
                blk["wp"], blk["w2"] = blk["proj"].w, blk["fc2"].w
            blk["bp"], blk["b2"] = f32(p + "attn.proj.bias"), f32(p + "mlp.fc2.bias")
            self.blocks.append(blk)
        self.post_ln = (g("post_ln.weight"), g("post_ln.bias"))
        self.w_lm, self.b_lm = g("lm_head.weight"), f32("lm_head.bias")
        self.cs = freqs_cis(c["rot"], max(ctx, 2048), c["theta"]).to(dev).contiguous()
        self.kc = [torch.zeros(self.nq, self.H, ctx, self.hd, device=dev, dtype=BF) for _ in self.blocks]
        self.vc = [torch.zeros(self.nq, self.H, ctx, self.hd, device=dev, dtype=BF) for _ in self.blocks]
        # ---- yes/no query state (md2fast.py:128-143)
        self.yes_ids, self.no_ids = list(yes_ids), list(no_ids)
        self.yn_ids = self.yes_ids + self.no_ids
        self.lm_small = None
        if self.yn_ids:
            npad = -(-len(self.yn_ids) // 4) * 4  # the GEMM wants N % 4 == 0: zero rows pad the head
            wy = torch.zeros(npad, self.D, device=dev, dtype=BF)
            by = torch.zeros(npad, device=dev, dtype=torch.float32)
            idx = torch.tensor(self.yn_ids, device=dev)
            wy[:len(self.yn_ids)] = self.w_lm[idx]
            by[:len(self.yn_ids)] = self.b_lm[idx]
            self.lm_small = ops.MxLin(wy, by, BF, dev)
        self.lm_full = None
        self.full_logits = False  # True: all V logits (the reference's diagnostics switch, md2fast.py:116)
        self.tok_buf = torch.zeros(self.nq, self.L, device=dev, dtype=torch.int64)
        self.last_idx = torch.zeros(self.nq, device=dev, dtype=torch.int64)
        self.prefix = None
        self.query_graph = None
        self.prefill_graph = None  # (graph, hidden-state output, image rows, prompt length) of capture_prefill
        self.fuse_ln = True  # fc2's reduction with the next layer's LayerNorm in one kernel where it pays
        # ---- decode-step device state
        lib = _lib.load()
        if not 1 <= attn_splits <= 8:
            raise ValueError(f"attn_splits {attn_splits} outside 1..8")
        # decode attention: workgroups per head (S > 1: their records merged by mx_gemv_res2). One is fastest at
        # contexts up to 1024 (1453 / 1364 / 1249 tok/s for 1 / 2 / 4): the merge costs more than it saves.
        self.S = attn_splits
        self.nparts = lib.mx_lm_argmax_nparts(self.V)
        self.part = torch.zeros(self.nparts, device=dev, dtype=torch.int64)
        self.state = torch.zeros(2, device=dev, dtype=torch.int32)
        self.tokens = torch.zeros(ctx, device=dev, dtype=torch.int32)
        self.xd = [torch.zeros(self.D, device=dev, dtype=BF) for _ in range(2)]
        self.qkv_d = torch.zeros(3 * self.D, device=dev, dtype=BF)
        self.g_d = torch.zeros(c["ff"], device=dev, dtype=BF)
        self.a_d = torch.zeros(self.D, device=dev, dtype=BF)
        self.y2_d = torch.zeros(self.D, device=dev, dtype=BF)  # bf16(fc2(g) + b2) of the decode step
        # decode: fc2 shares the attention's launch (mx_decode_attn_fc2) and proj + residual follow (mx_gemv_res2);
        # False: attention, then both GEMVs in one pass (mx_gemv_dual_res). Same roundings either way.
        self.fc2_with_attn = True
        self.attn_ws = torch.zeros(self.H * 8 * 66, device=dev, dtype=torch.float32)  # split records, S <= 8
        self.attn_cnt = torch.zeros(self.H, device=dev, dtype=torch.int32)
        self.logits = torch.zeros(self.V, device=dev, dtype=BF)
        self.pos_base = 0
        self.steps = 0
        self.graph = None
        # one launch per decode step (mx_decode_step_mk, or mx_decode_step_mk_i8 for the W8A8 Linears) where its
        # shapes hold: the 2048-wide, 32 x 64-head, 8192-MLP model, a cache of at most 1024 positions, one attention
        # split, and a device with a CU for each of its workgroups; the per-layer kernels above otherwise (use_mk =
        # False selects them too)
        self.mk_layers = self.mk_ll = self.mk_ep = None
        if (dev.type == "cuda" and attn_splits == 1 and (self.D, self.H, self.hd, c["ff"]) == (2048, 32, 64, 8192)
                and ctx <= 1024 and self.V <= 65536
                and torch.cuda.get_device_properties(dev).multi_processor_count >= lib.mx_decode_mk_grid()):
            self._init_mk()
        self.use_mk = self.mk_layers is not None
        self.mk_fallbacks = 0  # generations redone on the per-layer kernels after a one-launch step timed out

    def _init_mk(self):
        lib = _lib.load()
        rows = []
        for i, b in enumerate(self.blocks):
            for t, shape in ((b["wqf"], (3 * self.D + 8192, self.D)), (b["w2"], (self.D, 8192)), (b["wp"], (self.D, self.D))):
                if tuple(t.shape) != shape or not t.is_contiguous():
                    return
            scales = [b["sqf"].data_ptr(), b["sw2"].data_ptr(), b["swp"].data_ptr()] if self.w8a8 else [0, 0, 0]
            rows.append([b["ln"][0].data_ptr(), b["ln"][1].data_ptr(), b["wqf"].data_ptr(), b["bqf"].data_ptr(),
                         b["w2"].data_ptr(), b["b2"].data_ptr(), b["wp"].data_ptr(), b["bp"].data_ptr(),
                         self.kc[i].data_ptr(), self.vc[i].data_ptr()] + scales)
        if lib.mx_decode_mk_layer_bytes() != 8 * len(rows[0]):
            raise RuntimeError("layer descriptor size mismatch with the library")
        self.mk_layers = torch.tensor(rows, dtype=torch.int64).to(self.dev)
        self.mk_ll = torch.zeros(lib.mx_decode_mk_words(), dtype=torch.int64, device=self.dev)
        self.mk_ep = torch.zeros(2, dtype=torch.int32, device=self.dev)

    def mk_error(self):
        """The one-launch step's error word (0: every wait completed). Synchronises."""
        return 0 if self.mk_ep is None else int(self.mk_ep[1].item())

    def mk_reset(self):
        """Clear the exchange words and the epoch after a failed step."""
        if self.mk_ep is not None:
            self.mk_ll.zero_()
            self.mk_ep.zero_()

    # ------------------------------------------------------------------ prefill (md2fast.py:169-212)
    def _text_layers(self, x, pos0, causal_from, B=1, bcast=False):
        """x (B * n, D) bf16: B sequences (cache slots 0 .. B - 1) of n tokens at positions pos0 .. pos0 + n - 1;
        attends to keys 0 .. pos0 + n - 1 of its own slot (key j visible to query i iff j < causal_from or
        j <= pos0 + i; causal_from=None: all). bcast (B = 1): the K/V rows go to every cache slot (the shared image
        prefix, md2fast.py:177 rope_cache(..., bcast=(pos0 == 0)))."""
        n = x.shape[0] // B
        H, hd = self.H, self.hd
        Tk = pos0 + n
        h = None
        for i, b in enumerate(self.blocks):
            if h is None:
                h = ops.layernorm(x, *b["ln"], eps=self.eps)
            # W8A8: the LN output is quantised once for qkv and fc1 (SHARE_QUANT, md2fast.py:52, 174)
            pre = b["qkv"].quant(h) if self.w8a8 else None
            qkv = b["qkv"](h, pre=pre)
            q = torch.empty(B, H, n, hd, device=self.dev, dtype=BF)
            call("mx_rope_kv", stream(), qkv.data_ptr(), qkv.stride(0), self.cs.data_ptr(), q.data_ptr(),
                 self.kc[i].data_ptr(), self.vc[i].data_ptr(), B, n, H, self.ctx, pos0, self.nq, int(bcast))
            a = ops.sdpa(q, self.kc[i][:B, :, :Tk], self.vc[i][:B, :, :Tk], qpos0=pos0, causal_from=causal_from)
            r = b["proj"](a.view(B * n, self.D), res=x)
            f = b["fc1"](h, gelu=True, pre=pre)
            if i + 1 < len(self.blocks) and self._fuse_next_ln(b["fc2"], B * n):
                # fc2 as split-K partials, reduced with its bias and the residual by the kernel that also applies the
                # next layer's LayerNorm (one launch for the reduction and the norm)
                x, h = ops.residual_layernorm(b["fc2"].partial(f), b["fc2"].b, r, self.blocks[i + 1]["ln"],
                                              eps=self.eps)
            else:
                x, h = b["fc2"](f, res=r), None
        return x

    def _fuse_next_ln(self, lin, M):
        """fc2 + residual + the next layer's LayerNorm as partials + one row kernel: bf16 Linears whose row count has a
        partial GEMM pick in the tile table (the prefix and prefill passes; the yes/no query's 32-row fc2 keeps its 8
        raw splits, faster than 4 partial splits with the norm fused: the row kernel reads at most 4)."""
        return self.fuse_ln and hasattr(lin, "partial") and ops.has_partial_pick(M, lin)

    def prefill(self, img_emb, prompt_ids):
        """[BOS] + image tokens (mask-free, md2fast.py:201-206), then the prompt (prefix + causal mask,
        md2fast.py:208-212), as one pass over all n rows: every layer is row-wise except the attention, and one
        attention call with causal_from = P gives both parts their masks (key j is visible to query i iff j < P or
        j <= i: prefix queries see the prefix only, mask-free; prompt queries the prefix and the prompt up to
        themselves). All rows' K/V go into every cache slot (the prefix's must; the prompt rows in slots other than 0
        are rewritten by query() before it reads them). Leaves the first generated token's argmax in `part` and returns
        the prompt's hidden states.
        With a graph from capture_prefill() for these shapes, the inputs are copied into its buffers and it is replayed
        (the returned tensor is then the graph's output buffer, overwritten by the next replay)."""
        pg = self.prefill_graph
        if pg is not None and pg[2] == img_emb.shape[0] and pg[3] == prompt_ids.shape[0]:
            self._check_prefix(img_emb.shape[0])
            self.pf_img.copy_(img_emb)
            self.pf_ids.copy_(prompt_ids)
            pg[0].replay()
            self.prefix = 1 + img_emb.shape[0]
            self.pos_base = self.prefix + prompt_ids.shape[0]
            return pg[1]
        return self._prefill(img_emb, prompt_ids)

    def _prefill(self, img_emb, prompt_ids):
        self._check_prefix(img_emb.shape[0])
        P = 1 + img_emb.shape[0]
        x = torch.cat([self.wte[BOS:BOS + 1], img_emb.to(self.dev, BF), self.wte[prompt_ids.to(self.dev)]], dim=0)
        if x.shape[0] > self.ctx:
            raise ValueError(f"prefill of {x.shape[0]} tokens exceeds the cache ({self.ctx})")
        xp = self._text_layers(x, 0, P, bcast=True)[P:]
        self.prefix = P
        self.pos_base = x.shape[0]
        self.lm_argmax(xp[-1], logits=True)
        return xp

    def capture_prefill(self, n_img, n_prompt):
        """HIP graph of prefill() for n_img image rows and n_prompt prompt ids (the reference records its encode step
        the same way, md2fast.py:238-256): two eager warm-ups tune every GEMM shape outside capture, then the graph
        reads the fixed device buffers pf_img / pf_ids, which prefill() fills before each replay."""
        self._check_prefix(n_img)
        self.pf_img = torch.zeros(n_img, self.D, device=self.dev, dtype=BF)
        self.pf_ids = torch.zeros(n_prompt, device=self.dev, dtype=torch.int64)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self._prefill(self.pf_img, self.pf_ids)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = self._prefill(self.pf_img, self.pf_ids)
        torch.cuda.synchronize()
        self.prefill_graph = (g, out, n_img, n_prompt)
        return g

    def _check_prefix(self, n_img):
        if 1 + n_img + self.L > self.ctx:
            raise ValueError(f"prefix {1 + n_img} + L {self.L} exceeds the cache ({self.ctx})")

    def encode(self, img_emb):
        """Prefix prefill: [BOS] + image tokens, mask-free, K/V into every cache slot (md2fast.py:201-206).
        Returns the prefix length."""
        self._check_prefix(img_emb.shape[0])
        x = torch.cat([self.wte[BOS:BOS + 1], img_emb.to(self.dev, BF)], dim=0)
        self._text_layers(x, 0, None, bcast=True)
        self.prefix = x.shape[0]
        return self.prefix

    # ------------------------------------------------------------------ yes/no query (md2fast.py:208-212, 266-279)
    def set_questions(self, questions):
        """questions: nq token-id sequences (each 1 .. L ids, already templated). Zero-pads them to L and records
        each one's last row (md2fast.py:233-238)."""
        if len(questions) != self.nq:
            raise ValueError(f"{len(questions)} questions for nq = {self.nq}")
        buf = torch.zeros(self.nq, self.L, dtype=torch.int64)
        last = torch.zeros(self.nq, dtype=torch.int64)
        for b, q in enumerate(questions):
            ids = torch.as_tensor(q, dtype=torch.int64).flatten()
            if not 1 <= ids.numel() <= self.L:
                raise ValueError(f"question {b}: {ids.numel()} ids, need 1 .. {self.L}")
            if int(ids.min()) < 0 or int(ids.max()) >= self.V:
                raise ValueError(f"question {b}: token id outside [0, {self.V})")
            buf[b, :ids.numel()] = ids
            last[b] = b * self.L + ids.numel() - 1
        self.tok_buf.copy_(buf)
        self.last_idx.copy_(last)

    def _query(self):
        if self.prefix is None:
            raise RuntimeError("encode() the image prefix before querying")
        P = self.prefix
        x = self.wte[self.tok_buf.view(-1)]                                   # (nq * L, D)
        x = self._text_layers(x, P, P, B=self.nq)
        h = ops.layernorm(x.index_select(0, self.last_idx), *self.post_ln, eps=self.eps)  # (nq, D)
        if self.full_logits:
            if self.lm_full is None:
                self.lm_full = ops.MxLin(self.w_lm, self.b_lm, BF, self.dev)  # shares the LM-head storage
            return self.lm_full(h)
        if self.lm_small is None:
            raise RuntimeError("no yes/no ids were given: set full_logits or pass yes_ids / no_ids")
        return self.lm_small(h)[:, :len(self.yn_ids)]

    def query(self):
        """(nq, n_yes + n_no) logits of the yes / no rows, or (nq, V) with full_logits; the captured graph when
        there is one (md2fast.py:262-265)."""
        if self.query_graph is not None:
            self.query_graph[0].replay()
            return self.query_graph[1]
        return self._query()

    def capture_query(self):
        """HIP graph of the query for the current prefix length (md2fast.py:238-256): replays read tok_buf /
        last_idx, so set_questions() between replays changes the questions."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self._query()  # tunes every shape before capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = self._query()
        torch.cuda.synchronize()
        self.query_graph = (g, out)
        return g

    def decide(self, logits):
        """Per question (pred_yes, argmax id or -1, margin), margin = logsumexp(yes) - logsumexp(no) in fp32
        (md2fast.py:270-279): -1 when only the yes / no rows were computed."""
        lg = logits.float()
        if lg.dim() == 1:
            lg = lg[None]
        ny = len(self.yes_ids)
        out = []
        for r in lg:
            if r.numel() == len(self.yn_ids):
                m, am = (torch.logsumexp(r[:ny], 0) - torch.logsumexp(r[ny:], 0)).item(), -1
            else:
                m = (torch.logsumexp(r[self.yes_ids], 0) - torch.logsumexp(r[self.no_ids], 0)).item()
                am = int(r.argmax().item())
            out.append((m > 0, am, m))
        return out

    def lm_argmax(self, x_row, logits=False):
        call("mx_ln_gemv_argmax", stream(), x_row.data_ptr(), self.post_ln[0].data_ptr(), self.post_ln[1].data_ptr(),
             float(self.eps), self.w_lm.data_ptr(), self.w_lm.stride(0), self.b_lm.data_ptr(), self.V, self.D,
             ptr(self.logits) if logits else None, self.part.data_ptr(), self.nparts)

    # ------------------------------------------------------------------ decode
    def _check_room(self, pos_base, n_tokens):
        """n_tokens generated from a prefill that ends at pos_base - 1 need n_tokens - 1 decode steps at positions
        pos_base .. pos_base + n_tokens - 2, all below ctx."""
        if n_tokens < 1 or pos_base + n_tokens - 1 > self.ctx:
            raise ValueError(f"{n_tokens} tokens after a {pos_base}-token prefill exceed the {self.ctx}-entry KV cache")

    def start_decode(self):
        """Reset the step counter and feed the prefill's argmax token (becomes tokens[0])."""
        self.state.zero_()
        self.steps = 0
        self._embed()

    def _embed(self):
        # cap: steps the cache holds beyond the prefill (+ 1 for the prefill's own token), so the device state can
        # never index past the cache or tokens[] even if a step the host allowed ran once too often
        cap = max(1, min(self.ctx - self.pos_base + 1, self.ctx))
        call("mx_embed_step", stream(), self.part.data_ptr(), self.nparts, self.wte.data_ptr(), self.D,
             self.state.data_ptr(), self.pos_base, self.tokens.data_ptr(), cap, self.xd[0].data_ptr())

    def _count_step(self):
        """Host count of the decode steps since start_decode (the device state is never read back): refuse a step
        whose position would fall outside the cache."""
        if self.pos_base + self.steps >= self.ctx:
            raise ValueError(f"decode step at position {self.pos_base + self.steps} is past the {self.ctx}-entry cache")
        self.steps += 1

    def replay_step(self):
        """One decode step by graph replay (captured with capture_step), with the same capacity check."""
        self._count_step()
        self.graph.replay()

    def decode_step(self, logits=False):
        """One greedy step for the token in xd[0] at position state[1]: appends its K/V, computes the next token's
        argmax and embeds it into xd[0]. Graph-capturable (no host reads)."""
        if not torch.cuda.is_current_stream_capturing():
            self._count_step()
        st = stream()
        lib = _lib.load()
        if self.use_mk:
            cap = max(1, min(self.ctx - self.pos_base + 1, self.ctx))
            fn = lib.mx_decode_step_mk_i8 if self.w8a8 else lib.mx_decode_step_mk
            _lib.check(fn(st, self.mk_layers.data_ptr(), len(self.blocks), self.ctx,
                                             self.post_ln[0].data_ptr(), self.post_ln[1].data_ptr(),
                                             self.w_lm.data_ptr(), self.b_lm.data_ptr(), self.V, self.wte.data_ptr(),
                                             self.cs.data_ptr(), float(self.eps), float(self.hd ** -0.5),
                                             self.xd[0].data_ptr(), self.state.data_ptr(), self.pos_base,
                                             self.tokens.data_ptr(), cap, ptr(self.logits) if logits else None,
                                             self.mk_ll.data_ptr(), self.mk_ep.data_ptr()), "mx_decode_step_mk")
            return
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
            if self.fc2_with_attn:
                self._attn_fc2_res(b, i, x, xn)
                xi ^= 1
                continue
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

    def _attn_fc2_res(self, b, i, x, xn):
        """Layer i's attention with the fc2 GEMV in the same launch (it reads only the fc1 output), then proj +
        the parallel residual: xn = bf16(bf16(fc2(g) + b2) + bf16(bf16(proj(a) + bp) + x)) (md2fast.py:198)."""
        st, lib = stream(), _lib.load()
        S, part = self.S, self.attn_ws.data_ptr()
        attn = (st, self.qkv_d.data_ptr(), self.cs.data_ptr(), self.kc[i].data_ptr(), self.vc[i].data_ptr(), self.H,
                self.ctx, self.state.data_ptr(), float(self.hd ** -0.5), S, part, self.a_d.data_ptr(),
                self.g_d.data_ptr())
        att = (self.y2_d.data_ptr(), self.a_d.data_ptr(), S, part)
        if self.w8a8:
            _lib.check(lib.mx_decode_attn_fc2_i8(*attn, b["w2"].data_ptr(), b["sw2"].data_ptr(), b["b2"].data_ptr(),
                                                 b["w2"].shape[1], self.y2_d.data_ptr(), self.D),
                       "mx_decode_attn_fc2_i8")
            _lib.check(lib.mx_gemv_res2_i8(st, *att, b["wp"].data_ptr(), b["swp"].data_ptr(), b["bp"].data_ptr(),
                                           b["wp"].shape[1], x.data_ptr(), xn.data_ptr(), self.D), "mx_gemv_res2_i8")
        else:
            _lib.check(lib.mx_decode_attn_fc2(*attn, b["w2"].data_ptr(), b["b2"].data_ptr(), b["w2"].shape[1],
                                              self.y2_d.data_ptr(), self.D), "mx_decode_attn_fc2")
            _lib.check(lib.mx_gemv_res2(st, *att, b["wp"].data_ptr(), b["bp"].data_ptr(), b["wp"].shape[1],
                                        x.data_ptr(), xn.data_ptr(), self.D), "mx_gemv_res2")

    def capture_step(self):
        """HIP graph of one decode step (the state counter makes each replay the next token)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.decode_step()
        self.graph = g
        return g

    def generate(self, img_emb, prompt_ids, n_tokens, use_graph=True):
        """Prefill + greedy decode; returns the n_tokens generated ids (the first comes from the prompt prefill).
        Raises ValueError, before any work, when the prefill plus n_tokens - 1 decode steps would not fit the cache."""
        self._check_room(1 + img_emb.shape[0] + prompt_ids.shape[0], n_tokens)
        self._generate(img_emb, prompt_ids, n_tokens, use_graph)
        if self.use_mk and self.mk_error():
            # a one-launch step's wait timed out (e.g. another process held CUs, so its 256 workgroups were not all
            # resident): its tokens and the cache rows it wrote are undefined. Clear the exchange words and redo the
            # whole generation on the per-layer kernels, which have no cross-workgroup waits.
            err = self.mk_error()
            self.mk_reset()
            self.mk_fallbacks += 1
            warnings.warn(f"one-launch decode step timed out (error {err}); regenerating on the per-layer kernels")
            self.use_mk, self.graph = False, None
            try:
                self._generate(img_emb, prompt_ids, n_tokens, use_graph)
            finally:
                self.use_mk, self.graph = True, None
        return self.tokens[:n_tokens]

    def _generate(self, img_emb, prompt_ids, n_tokens, use_graph):
        self.prefill(img_emb, prompt_ids)
        self.start_decode()
        if use_graph:
            if self.graph is None:
                self.capture_step()  # recording does not execute the step
            for _ in range(n_tokens - 1):
                self.replay_step()
        else:
            for _ in range(n_tokens - 1):
                self.decode_step()
