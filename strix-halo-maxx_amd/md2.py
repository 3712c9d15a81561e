"""moondream2 per-model forwards on the MI355X kernels: the SigLIP vision tower (this file) and the text decoder
(md2text.py).

Structure follows the reference's FastMD2 (moondream/gpu/md2fast.py:70-287): the same block loop, the same
`lin_cls` plug-in point for the Linear class, `_vision` as the tower body, `capture()` for HIP-graph replay. The
differences are MI355X-side only:
  * any batch of crops (the reference runs batch 1), stacked as (B * 729) token rows so every GEMM sees M = B * 729;
  * the input normalisation + patchify is one kernel writing the patch-embedding GEMM's operand directly (K padded
    588 -> 592), and the position embedding is added in that GEMM's epilogue (broadcast over the batch);
  * q, k, v are read by the attention kernel straight out of the fused qkv GEMM output (strided views, no copies),
    and the attention output is written in (token, head * 72) order, i.e. already "transposed back";
  * residual adds and GELU run in the GEMM epilogues (the reference's fused_gelu / fused_res flags); with the
    library's own Linear (MxLin), the two residual Linears of a block (attention proj, MLP fc2) instead run split-K
    into fp32 partials, and one kernel adds the partials, bias and residual and applies the LayerNorm that reads the
    result (ln2, the next block's ln1, or the final post-LN), so each residual stream row is finished and
    normalised in a single pass.
"""
import torch

from . import ops
from .synth import VIS

BF = torch.bfloat16


class VisionTower:
    """SigLIP so400m tower: patch-embed + pos -> `layers` pre-LN blocks -> post-LN [-> projection MLP]."""

    def __init__(self, weights, lin_cls=ops.MxLin, device="cuda", attn=None):
        c = VIS
        self.dev = torch.device(device)
        self.D, self.H, self.hd, self.P, self.G = c["dim"], c["heads"], c["hd"], c["patch"], c["grid"]
        self.T = self.G * self.G
        self.eps = c["ln_eps"]
        g = lambda n: weights[n].to(self.dev, BF).contiguous()
        lin = lambda n: lin_cls(weights[n + ".weight"], weights[n + ".bias"], BF)
        self.patch_emb = lin("patch_emb")
        self.pos_emb = g("pos_emb").view(self.T, self.D)
        n = 0
        while f"blocks.{n}.ln1.weight" in weights:
            n += 1
        self.blocks = [dict(ln1=(g(f"blocks.{i}.ln1.weight"), g(f"blocks.{i}.ln1.bias")), qkv=lin(f"blocks.{i}.attn.qkv"),
                            proj=lin(f"blocks.{i}.attn.proj"), ln2=(g(f"blocks.{i}.ln2.weight"), g(f"blocks.{i}.ln2.bias")),
                            fc1=lin(f"blocks.{i}.mlp.fc1"), fc2=lin(f"blocks.{i}.mlp.fc2")) for i in range(n)]
        self.post_ln = (g("post_ln.weight"), g("post_ln.bias"))
        self.has_proj = "proj_mlp.fc1.weight" in weights
        if self.has_proj:
            self.proj_fc1, self.proj_fc2 = lin("proj_mlp.fc1"), lin("proj_mlp.fc2")
        self.attn = attn or ops.Attn(self.H, self.T, self.hd)
        self.graphs = {}
        # split-K residual Linears + fused residual LayerNorm when the Linear class can emit raw partial sums and the
        # batch is small (a few crops: too few output tiles to fill the GPU otherwise; large batches have enough
        # tiles, and there the fp32 partials would only add traffic)
        self.splitk = hasattr(self.blocks[0]["proj"], "partial") if self.blocks else False
        self.splitk_max_rows = 8192
        # which residual Linears run with their LayerNorm fused in (one launch instead of two) where the grid fits: the
        # attention projection (1152 x 1152, 64 x 64 tiles: 8.4 + 4.9 us -> one launch, 16-19 us less per frame). fc2
        # would need its 4304-deep k loop on 64 x 64 tiles without split-K, slower than its split-K GEMM plus the
        # separate residual LayerNorm (2.31 against 2.21 ms per frame), so it keeps the two launches.
        self.fuse_res_ln = {"proj"}

    def _attn(self, b, h, B):
        T, H, hd, D = self.T, self.H, self.hd, self.D
        qkv = b["qkv"](h)                                   # (B*T, 3D)
        q5 = qkv.view(B, T, 3, H, hd)
        q, k, v = (q5[:, :, i].transpose(1, 2) for i in range(3))   # (B, H, T, hd) strided views
        return self.attn(q, k, v).view(B * T, D)            # (B*T, D)

    def _fuse(self, lin, B, which):
        return (which in self.fuse_res_ln and hasattr(lin, "res_ln")
                and ops.res_ln_fits(B * self.T, lin.N, self.dev))

    def _block_sk(self, b, x, h, B, next_ln):
        """Split-K form of one block: x (residual stream) and h = ln1(x) in; the block output and next_ln(output)
        out (the second is None when next_ln is None). Where the grid fits (a few crops), a residual Linear and the
        LayerNorm after it are one launch (MxLin.res_ln)."""
        a = self._attn(b, h, B)
        if self._fuse(b["proj"], B, "proj"):
            x1, h2 = b["proj"].res_ln(a, x, b["ln2"], eps=self.eps)
        else:
            x1, h2 = ops.residual_layernorm(b["proj"].partial(a), b["proj"].b, x, b["ln2"], eps=self.eps)
        f = b["fc1"](h2, gelu=True)
        if next_ln is not None and self._fuse(b["fc2"], B, "fc2"):
            return b["fc2"].res_ln(f, x1, next_ln, eps=self.eps)
        return ops.residual_layernorm(b["fc2"].partial(f), b["fc2"].b, x1, next_ln, eps=self.eps)

    def rln_error(self):
        """Non-zero if a fused residual-LayerNorm launch timed out waiting for its row block (results undefined).
        Synchronises."""
        return ops.RlnWorkspace.device_error(self.dev)

    def check(self):
        """Raise if a fused residual-LayerNorm launch since the last reset timed out (its outputs are undefined),
        after zeroing the words so the next call starts clean. One small device read (synchronises)."""
        err = self.rln_error()
        if err:
            ops.RlnWorkspace.reset_device(self.dev)
            raise RuntimeError(f"fused residual-LayerNorm GEMM: a row-block wait timed out (error {err}); the last "
                               "tower outputs are undefined")

    # ---- one pre-LN block (md2fast.py:152-157)
    def _use_splitk(self, B):
        return self.splitk and B * self.T <= self.splitk_max_rows

    def block(self, b, x, B):
        h = ops.layernorm(x, *b["ln1"], eps=self.eps)
        if self._use_splitk(B):
            return self._block_sk(b, x, h, B, None)[0]
        x = b["proj"](self._attn(b, h, B), res=x)
        return b["fc2"](b["fc1"](ops.layernorm(x, *b["ln2"], eps=self.eps), gelu=True), res=x)

    def embed(self, img_u8):
        B = img_u8.shape[0]
        a = ops.patchify(img_u8, self.P, mode=0, ldo=self.patch_emb.Kp)        # (B*T, 592)
        return self.patch_emb(a, res=self.pos_emb)                            # (B*T, D), + pos_emb per image

    def _vision(self, img_u8, project=None):
        """img_u8 (B, 378, 378, 3) uint8 on the device -> (B, 729, 1152) post-LN features
        (or (B, 729, 2048) after the projection MLP when project=True)."""
        B = img_u8.shape[0]
        x = self.embed(img_u8)
        if self._use_splitk(B):
            h = ops.layernorm(x, *self.blocks[0]["ln1"], eps=self.eps)
            for i, b in enumerate(self.blocks):
                nxt = self.blocks[i + 1]["ln1"] if i + 1 < len(self.blocks) else self.post_ln
                x, h = self._block_sk(b, x, h, B, nxt)
            x = h
        else:
            for b in self.blocks:
                x = self.block(b, x, B)
            x = ops.layernorm(x, *self.post_ln, eps=self.eps)
        if project:
            x = self.project(x)
        return x.view(B, self.T, -1)

    def project(self, x):
        """Projection MLP on cat([x, x]) (md2fast.py:159-160): the global crop doubles as the local crop at 378x378."""
        feats = torch.cat([x, x], dim=-1)
        return self.proj_fc2(self.proj_fc1(feats, gelu=True))

    __call__ = _vision

    # ---- HIP-graph capture of the whole tower for a fixed input buffer (md2fast.py:238-256)
    def capture(self, img_buf):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self._vision(img_buf)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.check()  # the eager warm-up runs finished without a timed-out wait
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = self._vision(img_buf)
        torch.cuda.synchronize()
        self.graphs[img_buf.data_ptr()] = (g, out)
        return g, out
