"""TAPNext-style TRecViT on the MI355X kernels: per-frame streaming step (the model.step(frame, queries, caches)
contract, tapnext/npu/davis_cpu.py:78) and a clip-parallel form that runs F frames through each block at once with
the RG-LRU recurrence as a time scan.

Block (tapnext/npu/step8.py:470-488):
    t0 = RMSNorm(x); [y | xx] = linear_yx(t0); yg = gelu_tanh(y)
    xc = conv_1d(xx over frames t-3..t); xl = RG-LRU(xc, h); hh = linear_out(xl * yg); res = hh + x
    x1 = ffw_down(gelu_tanh(gate) * up) + res, [gate | up] = ffw_up(RMSNorm(res))
    x2 = x1 + out_proj(MHA(LN(x1)))  (12 heads x 64, scale 1/8, non-causal over all tokens of the frame)
    x3 = x2 + mlp3(gelu_erf(mlp0(LN(x2))))
then encoder_norm after the last block.

Kernel mapping (per block, one frame = 1280 tokens):
    RMSNorm -> GEMM yx (GELU on the y columns only, output straight into this frame's slot of a 4-frame ring: the
    conv reads its history from the ring, nothing is copied) -> fused conv + gates + RG-LRU + y-gate (mx_ssm_step)
    -> GEMM out (+x) -> RMSNorm -> GEMM up with the gated-GELU epilogue (weight rows interleaved gate/up at load
    time) -> GEMM down (+res) -> LN -> GEMM qkv -> fused SDPA -> GEMM out_proj (+x1) -> LN -> GEMM mlp0 (GELU erf)
    -> GEMM mlp3 (+x2). A frame is one HIP graph per ring phase (4 graphs), with the frame counter in device memory.
Inputs per frame: patch conv 8x8/8 of the frame resized to 256 x 256 (bilinear) and normalised by /127.5 - 1
(one resize + patchify kernel, or the plain patchify kernel for a frame already at 256, then a GEMM with the
position embedding added in the epilogue) and 256 query tokens from a linear embedding of the (y, x) coordinates / 256 (a stand-in:
the real embed_queries lives in the external model and is not part of the block).
Outputs per frame (model.step's tracks, logits, vis; tapnext/npu/step8.py:327-362): the coordinate and visibility
heads on the encoder-normed query tokens plus the windowed soft-argmax readout, one fp32 kernel (mx_track_heads)
at the end of the frame's graph.
"""
import math

import torch

from . import _lib, ops
from ._lib import call, ptr, stream
from .synth import TRV

BF = torch.bfloat16


def _head_blob(weights, name, dev):
    """One head's fp32 weight blob in the kernel's layout: W0^T | b0 | g1 | beta1 | W3^T | b3 | g4 | beta4 | W6^T | b6
    (nn.Sequential indices: 0 / 3 / 6 Linear, 1 / 4 LayerNorm)."""
    W = lambda i: weights[f"{name}.{i}.weight"].float()
    B = lambda i: weights[f"{name}.{i}.bias"].float()
    parts = [W(0).t(), B(0), W(1), B(1), W(3).t(), B(3), W(4), B(4), W(6).t(), B(6)]
    return torch.cat([t.contiguous().reshape(-1) for t in parts]).to(dev)


def _interleave_rows(w, b):
    """ffw_up [gate (F) | up (F)] rows -> (gate_0, up_0, gate_1, up_1, ...) for the gated-GELU epilogue."""
    F = w.shape[0] // 2
    wi = torch.stack([w[:F], w[F:]], dim=1).reshape(2 * F, -1)
    bi = torch.stack([b[:F], b[F:]], dim=1).reshape(2 * F)
    return wi, bi


class RGLRU:
    """TAPNext's RG-LRU layer on its own, the interface the reference swaps numerics at:
    RGLRU.forward(x, h0) -> (y, h) (tapnext/npu/r9/cpuemu.py:33-47, monkey-patched in at :110-116), one launch of
    mx_rglru_step. x: bf16 (..., C), the layer's input (the temporal conv's output); h0: fp32 (..., C) state or None
    on a video's first frame (then h = x * sigmoid(gate_x)); returns y = bf16(h) and h fp32, both new tensors of x's
    shape. Parameters as the module holds them: input_gate / a_gate BlockDiagonalLinear weights (H, 64, 64) (in, out)
    and biases (H, 64), a_param (C,)."""

    def __init__(self, input_gate_w, input_gate_b, a_gate_w, a_gate_b, a_param, device="cuda"):
        dev = torch.device(device)
        H, bi, bo = input_gate_w.shape
        if (bi, bo) != (64, 64) or tuple(a_gate_w.shape) != (H, 64, 64):
            raise ValueError("block-diagonal gates must be (H, 64, 64)")
        self.C = 64 * H
        bf = lambda t: t.detach().to(dev, BF).contiguous()
        self.wxT = bf(input_gate_w.transpose(-1, -2))   # [head][out][in]
        self.waT = bf(a_gate_w.transpose(-1, -2))
        self.bx = bf(input_gate_b.reshape(-1))
        self.ba = bf(a_gate_b.reshape(-1))
        # bf16(softplus(a_param)) from the exact value (F.softplus on the module's parameter, rounded once)
        self.sp = torch.log1p(torch.exp(a_param.detach().double().cpu())).to(BF).to(dev).contiguous()

    def forward(self, x, h0=None):
        C = self.C
        if x.shape[-1] != C:
            raise ValueError(f"input width {x.shape[-1]} != {C}")
        x2 = x.reshape(-1, C)
        if x2.dtype != BF or x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.to(BF).contiguous()
        T = x2.shape[0]
        h = torch.empty(T, C, device=x2.device, dtype=torch.float32)
        y = torch.empty(T, C, device=x2.device, dtype=BF)
        hp = None
        if h0 is not None:
            if h0.shape != x.shape:
                raise ValueError(f"h0 {tuple(h0.shape)} != x {tuple(x.shape)}")
            hp = h0.reshape(T, C).to(torch.float32).contiguous()
        call("mx_rglru_step", stream(), x2.data_ptr(), x2.stride(0), ptr(hp), self.wxT.data_ptr(), self.bx.data_ptr(),
             self.waT.data_ptr(), self.ba.data_ptr(), self.sp.data_ptr(), h.data_ptr(), y.data_ptr(), C, T, C)
        return y.view(x.shape), h.view(x.shape)

    __call__ = forward


def rglru_step(x, h0, params):
    """(y bf16, h fp32) = the RG-LRU layer on x with state h0 (None: first frame); params: an RGLRU, or a dict with
    the module's tensors (input_gate_w, input_gate_b, a_gate_w, a_gate_b, a_param)."""
    layer = params if isinstance(params, RGLRU) else RGLRU(device=x.device, **params)
    return layer(x, h0)


class TRecViT:
    def __init__(self, weights, n_tokens=None, device="cuda", lin_cls=ops.MxLin):
        c = TRV
        self.dev = dev = torch.device(device)
        self.D, self.H, self.hd = c["dim"], c["heads"], c["hd"]
        self.P = c["patch"]
        self.G = c["img"] // self.P
        self.n_img = self.G * self.G
        self.n_q = c["n_q"]
        self.T = self.n_img + self.n_q if n_tokens is None else n_tokens
        self.rms_eps, self.ln_eps = c["rms_eps"], c["ln_eps"]
        g = lambda n: weights[n].to(dev, BF).contiguous()
        lin = lambda n, wn=None, bn=None: lin_cls(weights[wn or n + ".weight"], weights[bn or n + ".bias"], BF)
        n = 0
        while f"blocks.{n}.ssm_block.temporal_pre_norm.scale" in weights:
            n += 1
        self.blocks = []
        for i in range(n):
            rb = f"blocks.{i}.ssm_block.recurrent_block."
            mb = f"blocks.{i}.ssm_block.mlp_block."
            vb = f"blocks.{i}.vit_block."
            sb = f"blocks.{i}.ssm_block."
            sc1 = lambda k: (weights[k].float() + 1).to(BF).to(dev).contiguous()  # torch: 1 + scale in bf16
            wu, bu = _interleave_rows(weights[mb + "ffw_up.weight"], weights[mb + "ffw_up.bias"])
            ap = weights[rb + "rg_lru.a_param"].double()
            blk = dict(
                sc0=sc1(sb + "temporal_pre_norm.scale"), sc1=sc1(sb + "channel_pre_norm.scale"),
                yx=lin(rb + "linear_yx"), out=lin(rb + "linear_out"),
                up=lin_cls(wu, bu, BF), down=lin(mb + "ffw_down"),
                ln1=(g(vb + "ln_1.weight"), g(vb + "ln_1.bias")), ln2=(g(vb + "ln_2.weight"), g(vb + "ln_2.bias")),
                qkv=lin(None, vb + "self_attention.in_proj_weight", vb + "self_attention.in_proj_bias"),
                oproj=lin(vb + "self_attention.out_proj"), mlp0=lin(vb + "mlp.0"), mlp3=lin(vb + "mlp.3"),
                conv_w=g(rb + "conv_1d.w"), conv_b=g(rb + "conv_1d.b"),
                wxT=weights[rb + "rg_lru.input_gate.w"].transpose(-1, -2).to(dev, BF).contiguous(),
                bx=weights[rb + "rg_lru.input_gate.b"].reshape(-1).to(dev, BF).contiguous(),
                waT=weights[rb + "rg_lru.a_gate.w"].transpose(-1, -2).to(dev, BF).contiguous(),
                ba=weights[rb + "rg_lru.a_gate.b"].reshape(-1).to(dev, BF).contiguous(),
                # pack8.py:141-142 / ssm_ref: sp = bf16(softplus(a_param)), computed in fp64
                sp=torch.log1p(torch.exp(ap)).to(BF).to(dev).contiguous(),
            )
            self.blocks.append(blk)
        self.enc_norm = (g("encoder_norm.weight"), g("encoder_norm.bias"))
        self.patch = lin_cls(weights["lin_proj.weight"].reshape(self.D, -1), weights["lin_proj.bias"], BF)
        self.pos = g("image_pos_emb").view(self.n_img, self.D)
        self.qproj = lin_cls(weights["query_proj.weight"], weights["query_proj.bias"], BF)
        # ---- tracking heads (optional: a weight dict without them yields tokens only)
        self.has_heads = "coordinate_head.0.weight" in weights
        if self.has_heads:
            lib = _lib.load()
            Hh = weights["coordinate_head.0.weight"].shape[0]
            self.NOC = weights["coordinate_head.6.weight"].shape[0]
            self.cblob = _head_blob(weights, "coordinate_head", dev)
            self.vblob = _head_blob(weights, "visible_head", dev)
            if (self.cblob.numel() != lib.mx_track_head_blob_elems(self.D, Hh, self.NOC)
                    or self.vblob.numel() != lib.mx_track_head_blob_elems(self.D, Hh, 1)):
                raise ValueError("head weights do not match Linear(D, H) / LayerNorm(H) / Linear(H, H) / Linear(H, NO)")
            self.Hh, self.head_eps, self.radius = Hh, c["head_ln_eps"], c["head_radius"]
            self.tracks = torch.zeros(self.n_q, 2, device=dev, dtype=torch.float32)
            self.logits = torch.zeros(self.n_q, self.NOC, device=dev, dtype=torch.float32)
            self.vis = torch.zeros(self.n_q, device=dev, dtype=torch.float32)
        # ---- streaming state: per block a 4-frame ring of [yg | xx] rows and the fp32 RG-LRU state
        T, D = self.T, self.D
        self.ring = [[torch.zeros(T, 2 * D, device=dev, dtype=BF) for _ in range(4)] for _ in self.blocks]
        self.h = [torch.zeros(T, D, device=dev, dtype=torch.float32) for _ in self.blocks]
        self.frame = torch.zeros(1, device=dev, dtype=torch.int32)
        self.x0 = torch.zeros(T, D, device=dev, dtype=BF)
        self.img = torch.zeros(c["img"], c["img"], 3, device=dev, dtype=torch.uint8)
        self.qfeat = torch.zeros(self.n_q, 2, device=dev, dtype=BF)
        self.t = 0  # host copy of the frame index (selects the ring phase)
        self.graphs = {}
        self.out = None
        # residual Linears whose epilogue runs as split-K fp32 partials + one row kernel that adds them, the bias and
        # the residual and applies the norm that reads the result (the next block's temporal pre-norm or the encoder
        # norm for mlp3): the two 3072-deep ones, whose 64 x 64 tiles otherwise stream 3072-wide rows per workgroup
        # (N = 768 leaves too few output tiles for larger ones). At most splitk_max_rows rows: larger batches (the
        # clip form) have enough tiles, and there the fp32 partials would only add traffic.
        self.fuse_norm = {"down", "mlp3"}
        self.splitk_max_rows = 8192
        # residual Linears whose norm runs inside the GEMM's own launch (MxLin.res_ln / res_rms: the tiles of a row
        # block exchange row statistics) where the grid fits one tile per CU (one frame: 20 x 12 tiles of 64 x 64):
        # linear_out with channel_pre_norm (RMSNorm), the attention out-projection with ln_2 (LayerNorm)
        self.fuse_rln = {"out", "oproj"}

    def reset(self):
        """A new video: zero every block's conv history and RG-LRU state and mark the next frame first
        (Step8.reset, tapnext/npu/step8.py:244-249)."""
        for rs in self.ring:
            for r in rs:
                r.zero_()
        for h in self.h:
            h.zero_()
        self.frame.zero_()
        self.t = 0

    # ------------------------------------------------------------------ per-frame input (X0)
    def embed(self, img_u8, qfeat, out):
        S = self.G * self.P
        if img_u8.shape[0] == S and img_u8.shape[1] == S:  # already at the model's size: the resize is the identity
            a = ops.patchify(img_u8[None], self.P, mode=1, ldo=self.patch.K)
        else:
            a = ops.resize_patchify(img_u8[None], S, self.P, ldo=self.patch.K)
        self.patch(a, res=self.pos, out=out[:self.n_img])
        self.qproj(qfeat, out=out[self.n_img:self.n_img + qfeat.shape[0]])
        return out

    # ------------------------------------------------------------------ one block, one frame
    def block_step(self, i, x, phase, t0=None, next_norm=None):
        """Block i on one streamed frame. t0: the block's temporal pre-norm of x when the previous block's tail
        already computed it (else computed here). next_norm: None returns the block output; ("rms", sc1) or
        ("ln", (gamma, beta)) returns (output, that norm of the output), the next block's temporal pre-norm or the
        encoder norm, fused into the last Linear's residual epilogue where it pays."""
        b = self.blocks[i]
        T, D = self.T, self.D
        ring = self.ring[i]
        cur = ring[phase]
        if t0 is None:
            t0 = ops.rmsnorm(x, b["sc0"], eps=self.rms_eps)
        b["yx"](t0, gelu=True, act_cols=D, out=cur)             # [gelu(y) | xx] into this frame's ring slot
        z = torch.empty(T, D, device=self.dev, dtype=BF)
        taps = [ring[(phase - k) % 4][:, D:] for k in range(4)]
        call("mx_ssm_step", stream(), *(t.data_ptr() for t in taps), 2 * D, cur.data_ptr(), 2 * D,
             b["conv_w"].data_ptr(), b["conv_b"].data_ptr(), b["wxT"].data_ptr(), b["bx"].data_ptr(),
             b["waT"].data_ptr(), b["ba"].data_ptr(), b["sp"].data_ptr(), self.frame.data_ptr(), self.h[i].data_ptr(),
             z.data_ptr(), D, T, D)
        return self._block_tail(b, z, x, 1, next_norm=next_norm)

    def _norm(self, x, norm):
        kind, p = norm
        if kind == "rms":
            return ops.rmsnorm(x, p, eps=self.rms_eps)
        return ops.layernorm(x, *p, eps=self.ln_eps)

    def _linres_norm(self, name, lin, a, res, norm):
        """x = lin(a) + res with torch's roundings and norm(x). The Linears in fuse_rln, where the grid fits one tile
        per CU, run as one launch with the norm (res_ln / res_rms). For those in fuse_norm (and at most
        splitk_max_rows rows) the GEMM writes split-K fp32 partials and one row kernel adds them, the bias and the
        residual and applies the norm; otherwise the GEMM's residual epilogue, then the norm kernel."""
        M = a.shape[0]
        if name in self.fuse_rln and hasattr(lin, "res_ln") and ops.res_ln_fits(M, lin.N, a.device):
            kind, p = norm
            if kind == "rms":
                return lin.res_rms(a, res, p, eps=self.rms_eps)
            return lin.res_ln(a, res, p, eps=self.ln_eps)
        if name in self.fuse_norm and M <= self.splitk_max_rows and hasattr(lin, "partial"):
            P = lin.partial(a)
            kind, p = norm
            if kind == "rms":
                return ops.residual_rmsnorm(P, lin.b, res, p, eps=self.rms_eps)
            return ops.residual_layernorm(P, lin.b, res, p, eps=self.ln_eps)
        x = lin(a, res=res)
        return x, self._norm(x, norm)

    def _block_tail(self, b, z, x, B, T=None, next_norm=None):
        T = self.T if T is None else T
        D, H = self.D, self.H
        res, t1 = self._linres_norm("out", b["out"], z, x, ("rms", b["sc1"]))
        g = b["up"](t1, act="glu")
        x1, h1 = self._linres_norm("down", b["down"], g, res, ("ln", b["ln1"]))
        qkv = b["qkv"](h1)
        q5 = qkv.view(B, T, 3, H, self.hd)
        q, k, v = (q5[:, :, j].transpose(1, 2) for j in range(3))
        a = ops.sdpa(q, k, v, scale=1.0 / 8.0)
        x2, h2 = self._linres_norm("oproj", b["oproj"], a.view(B * T, D), x1, ("ln", b["ln2"]))
        f = b["mlp0"](h2, act="erf")
        if next_norm is None:
            return b["mlp3"](f, res=x2)
        return self._linres_norm("mlp3", b["mlp3"], f, x2, next_norm)

    def _next_norm(self, i):
        """The norm applied to block i's output: the next block's temporal pre-norm, or the encoder norm."""
        return ("rms", self.blocks[i + 1]["sc0"]) if i + 1 < len(self.blocks) else ("ln", self.enc_norm)

    def heads(self, xq, tracks=None, logits=None, vis=None):
        """model.heads on the encoder-normed query rows xq (Q, D) bf16: tracks (Q, 2) fp32 (first-half / second-half
        readouts), coordinate logits (Q, NOC) fp32, visibility logits (Q,) fp32 (step8.py:327-362)."""
        Q = xq.shape[0]
        tracks = torch.empty(Q, 2, device=self.dev) if tracks is None else tracks
        logits = torch.empty(Q, self.NOC, device=self.dev) if logits is None else logits
        vis = torch.empty(Q, device=self.dev) if vis is None else vis
        e = float(self.head_eps)
        call("mx_track_heads", stream(), xq.data_ptr(), xq.stride(0), Q, self.D, self.Hh, self.cblob.data_ptr(),
             self.NOC, e, e, self.vblob.data_ptr(), e, e, self.radius, tracks.data_ptr(), logits.data_ptr(),
             logits.stride(0), vis.data_ptr())
        return tracks, logits, vis

    def _frame(self, phase):
        x = self.embed(self.img, self.qfeat, self.x0)
        t = ops.rmsnorm(x, self.blocks[0]["sc0"], eps=self.rms_eps) if self.blocks else None
        for i in range(len(self.blocks)):
            x, t = self.block_step(i, x, phase, t0=t, next_norm=self._next_norm(i))
        fin = t if self.blocks else ops.layernorm(x, *self.enc_norm, eps=self.ln_eps)
        if self.has_heads:
            self.heads(fin[self.n_img:self.n_img + self.n_q], self.tracks, self.logits, self.vis)
        call("mx_counter_add", stream(), self.frame.data_ptr(), 1)
        return fin

    def step(self, frame_u8, qfeat, use_graph=False):
        """One streamed frame: frame_u8 (H, W, 3) uint8 (resized to 256 x 256 on the device), qfeat (n_q, 2) ->
        encoder-normed tokens (T, D). The RG-LRU state and conv history advance (model.step)."""
        if self.img.shape != frame_u8.shape:  # a new frame size: new input buffer, and the graphs read the old one
            if frame_u8.dim() != 3 or frame_u8.shape[2] != 3:
                raise ValueError("frames are (H, W, 3) uint8")
            self.img = torch.zeros(frame_u8.shape, device=self.dev, dtype=torch.uint8)
            self.graphs = {}
        self.img.copy_(frame_u8, non_blocking=True)
        self.qfeat.copy_(qfeat, non_blocking=True)
        phase = self.t % 4
        if use_graph:
            if phase not in self.graphs:
                self.capture()
            g, out = self.graphs[phase]
            g.replay()
        else:
            out = self._frame(phase)
        self.t += 1
        return out

    def track(self, frame_u8, qfeat, use_graph=False):
        """model.step's outputs for one streamed frame (davis_cpu.py:78): (tracks, logits, vis), views of device
        buffers that the next frame overwrites."""
        if not self.has_heads:
            raise RuntimeError("the weights carry no tracking heads")
        self.step(frame_u8, qfeat, use_graph)
        return self.tracks, self.logits, self.vis

    def rln_ready(self):
        """Create the fused residual-LayerNorm GEMMs' statistics words (they cannot be allocated during capture)."""
        for name in self.fuse_rln:
            if self.blocks and hasattr(self.blocks[0][name], "res_ln"):
                ops.RlnWorkspace.get(self.dev, self.blocks[0][name].N)

    def rln_error(self):
        """Non-zero if a fused residual-LayerNorm launch timed out waiting for its row block (results undefined).
        Synchronises."""
        return ops.RlnWorkspace.device_error(self.dev)

    def capture(self):
        """One HIP graph per ring phase (kernel arguments differ only in which ring slots they read/write)."""
        self.rln_ready()
        for phase in range(4):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                out = self._frame(phase)
            self.graphs[phase] = (g, out)

    # ------------------------------------------------------------------ clip-parallel form
    def clip_state(self, F):
        """Buffers for F-frame clips: per block a stack of F + 3 frames of [yg | xx] rows (3 history frames first)."""
        T, D = self.T, self.D
        self.F = F
        self.stack = [torch.zeros(F + 3, T, 2 * D, device=self.dev, dtype=BF) for _ in self.blocks]
        self.Ab = torch.empty(F, T, D, device=self.dev, dtype=torch.float32)
        self.Bb = torch.empty(F, T, D, device=self.dev, dtype=torch.float32)

    def forward_clip(self, frames_u8, qfeat):
        """F frames at once through every block (GEMMs with M = F x T rows, attention batched over frames, the RG-LRU
        as a time scan). frames_u8 (F, H, W, 3) (resized to 256 x 256 on the device); returns (F, T, D). Continues
        from the stacked history / state."""
        F, T, D = frames_u8.shape[0], self.T, self.D
        x = torch.empty(F, T, D, device=self.dev, dtype=BF)
        for f in range(F):
            self.embed(frames_u8[f], qfeat, x[f])
        x = x.view(F * T, D)
        t0 = ops.rmsnorm(x, self.blocks[0]["sc0"], eps=self.rms_eps)
        for i, b in enumerate(self.blocks):
            st = self.stack[i]
            b["yx"](t0, gelu=True, act_cols=D, out=st[3:].view(F * T, 2 * D))
            xs = st[:, :, D:]
            call("mx_ssm_prep", stream(), xs.data_ptr(), 2 * D, T * 2 * D, b["conv_w"].data_ptr(), b["conv_b"].data_ptr(),
                 b["wxT"].data_ptr(), b["bx"].data_ptr(), b["waT"].data_ptr(), b["ba"].data_ptr(), b["sp"].data_ptr(),
                 self.frame.data_ptr(), self.Ab.data_ptr(), self.Bb.data_ptr(), F, T, D)
            z = torch.empty(F, T, D, device=self.dev, dtype=BF)
            call("mx_rglru_scan", stream(), self.Ab.data_ptr(), self.Bb.data_ptr(), self.h[i].data_ptr(), F, T, D,
                 st[3:].data_ptr(), 2 * D, T * 2 * D, z.data_ptr(), D, T * D)
            st[:3].copy_(st[F:F + 3])  # the last 3 frames become the next clip's history
            x, t0 = self._block_tail(b, z.view(F * T, D), x, F, next_norm=self._next_norm(i))
        fin = t0
        call("mx_counter_add", stream(), self.frame.data_ptr(), F)
        self.t += F
        return fin.view(F, T, D)


class CropTracker:
    """The TRecViT step over a moving n x n crop of the 32 x 32 patch grid with the recurrent state indexed by
    absolute patch (tapnext/crop-study/crop_study.py:147-185, CropTracker with shift=True): each crop token keeps its
    own slice of the position embedding, its RG-LRU state and conv history travel with the image content, tokens
    that leave the crop drop their state and tokens that enter start from zero. (The un-shifted form, state by
    crop-local slot, loses the tracks: common/book/negative-results.md F13.)

    Nothing is gathered or scattered per block: the SSM kernel addresses the model's absolute state rows through a
    row map (mx_ssm_step_rows), and per-row stamps in device memory say which state a row still has. The crop's
    tokens run every other op of the block as a T = n^2 + n_q token frame. Owns the model's state: do not interleave
    with TRecViT.step on the same model without a reset.
    """

    def __init__(self, model):
        m = self.m = model
        if m.T != m.n_img + m.n_q:
            raise ValueError("the crop form needs the full token layout (patch grid + queries)")
        dev, T, D = m.dev, m.T, m.D
        self.rows = torch.zeros(T, device=dev, dtype=torch.int32)
        self.stamps = torch.empty(2, T, 2, device=dev, dtype=torch.int32)
        self.xc = torch.zeros(T, D, device=dev, dtype=BF)
        self.cur = torch.zeros(T, 2 * D, device=dev, dtype=BF)
        self.graphs = {}
        self.reset()

    def reset(self):
        """A new video: zero the model's state and mark every state row as never in the crop."""
        self.m.reset()
        self.stamps.fill_(-8)

    def _row_map(self, r0, c0, n):
        G = self.m.G
        if not (1 <= n <= G and 0 <= r0 <= G - n and 0 <= c0 <= G - n):
            raise ValueError(f"crop ({r0}, {c0}, {n}) outside the {G} x {G} patch grid")
        ar = torch.arange(n)
        idx = ((r0 + ar)[:, None] * G + (c0 + ar)[None]).flatten()
        return torch.cat([idx, self.m.n_img + torch.arange(self.m.n_q)]).to(torch.int32)

    def _block(self, i, x, t0, phase, T):
        """Block i over the crop's T tokens; t0 = its temporal pre-norm of x. Returns (output, the next norm of it)."""
        m = self.m
        b, D, ring = m.blocks[i], m.D, m.ring[i]
        cur = self.cur[:T]
        b["yx"](t0, gelu=True, act_cols=D, out=cur)
        z = torch.empty(T, D, device=m.dev, dtype=BF)
        taps = [cur[:, D:]] + [ring[(phase - k) % 4][:, D:] for k in (1, 2, 3)]
        call("mx_ssm_step_rows", stream(), *(t.data_ptr() for t in taps), 2 * D, cur.data_ptr(), 2 * D,
             b["conv_w"].data_ptr(), b["conv_b"].data_ptr(), b["wxT"].data_ptr(), b["bx"].data_ptr(),
             b["waT"].data_ptr(), b["ba"].data_ptr(), b["sp"].data_ptr(), m.frame.data_ptr(), m.h[i].data_ptr(),
             z.data_ptr(), D, T, D, self.rows.data_ptr(), self.stamps.data_ptr(), m.T,
             ring[phase][:, D:].data_ptr(), 2 * D)
        return m._block_tail(b, z, x, 1, T, next_norm=m._next_norm(i))

    def _frame(self, phase, n):
        m = self.m
        T = n * n + m.n_q
        x = m.embed(m.img, m.qfeat, m.x0)  # the whole grid: a patch's embedding only depends on its own pixels
        xc = torch.index_select(x, 0, self.rows[:T], out=self.xc[:T])
        t = ops.rmsnorm(xc, m.blocks[0]["sc0"], eps=m.rms_eps)
        for i in range(len(m.blocks)):
            xc, t = self._block(i, xc, t, phase, T)
        fin = t
        if m.has_heads:
            m.heads(fin[n * n:], m.tracks, m.logits, m.vis)
        call("mx_counter_add", stream(), m.frame.data_ptr(), 1)
        return fin

    def step(self, frame_u8, qfeat, r0, c0, n, use_graph=False):
        """One frame over the crop of patch rows r0 .. r0 + n - 1, columns c0 .. c0 + n - 1 (patch units):
        returns the encoder-normed tokens (n^2 crop tokens, then the n_q query tokens)."""
        m = self.m
        if m.img.shape != frame_u8.shape:
            if frame_u8.dim() != 3 or frame_u8.shape[2] != 3:
                raise ValueError("frames are (H, W, 3) uint8")
            m.img = torch.zeros(frame_u8.shape, device=m.dev, dtype=torch.uint8)
            m.graphs, self.graphs = {}, {}
        m.img.copy_(frame_u8, non_blocking=True)
        m.qfeat.copy_(qfeat, non_blocking=True)
        rows = self._row_map(r0, c0, n)
        self.rows[:rows.numel()].copy_(rows)
        phase = m.t % 4
        if use_graph:
            if (phase, n) not in self.graphs:
                m.rln_ready()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    out = self._frame(phase, n)
                self.graphs[(phase, n)] = (g, out)
            g, out = self.graphs[(phase, n)]
            g.replay()
        else:
            out = self._frame(phase, n)
        m.t += 1
        return out

    def track(self, frame_u8, qfeat, r0, c0, n, use_graph=False):
        """(tracks, logits, vis) of the queries for one crop frame (full-frame coordinates, as the coordinate head
        always reads out full-frame bins)."""
        if not self.m.has_heads:
            raise RuntimeError("the weights carry no tracking heads")
        self.step(frame_u8, qfeat, r0, c0, n, use_graph)
        return self.m.tracks, self.m.logits, self.m.vis
