"""The whole moondream2 yes/no frame on the MI355X kernels: the reference's FastMD2 (moondream/gpu/md2fast.py:70-287)
composed from the vision tower (md2.py) and the text decoder (md2text.py).

    encode(img):  vision tower at batch 1 -> post-LN -> projection MLP on cat([x, x]) -> [BOS] + 729 image tokens
                  prefilled through the 24 text layers (mask-free), K/V into every question's cache slot
                  (md2fast.py:147-160, 201-206)
    query():      the nq questions (zero-padded to L ids) prefilled over the prefix under the prefix + causal mask,
                  the last real token of each through the final LN and the yes / no rows of the LM head
                  (md2fast.py:208-212)
    decide(...):  logsumexp(yes) - logsumexp(no) per question (md2fast.py:266-279)

capture() records encode and query as two HIP graphs (md2fast.py:238-256): encode reads the image from a fixed
device buffer, query reads the token buffer set_questions() writes, so frame(img) is two graph replays.
"""
import torch

from .md2 import VisionTower
from .md2text import TextDecoder

BF = torch.bfloat16


class FastMD2:
    def __init__(self, vision_weights, text_weights, device="cuda", nq=1, L=32, yes_ids=(), no_ids=(), w8a8=False,
                 ctx=None):
        """vision_weights must carry the projection MLP (proj_mlp.fc1 / fc2); yes_ids / no_ids are the token ids of
        the yes / no rows (the reference takes them from its tokenizer, md2fast.py:138-142)."""
        self.dev = torch.device(device)
        self.vt = VisionTower(vision_weights, device=self.dev)
        if not self.vt.has_proj:
            raise ValueError("the vision weights carry no projection MLP (proj_mlp.fc1 / proj_mlp.fc2)")
        n_prefix = 1 + self.vt.T
        ctx = ctx if ctx is not None else (n_prefix + L + 63) // 64 * 64
        self.td = TextDecoder(text_weights, device=self.dev, ctx=ctx, nq=nq, L=L, yes_ids=yes_ids, no_ids=no_ids,
                              w8a8=w8a8)
        S = self.vt.G * self.vt.P
        self.img = torch.zeros(S, S, 3, device=self.dev, dtype=torch.uint8)
        self.graphs = {}

    # ------------------------------------------------------------------ eager bodies
    def _encode(self):
        emb = self.vt._vision(self.img[None], project=True)[0]    # (729, 2048) projected image tokens
        return self.td.encode(emb)

    def encode(self, img_u8):
        """Image (378, 378, 3) uint8 -> the text prefix in the KV cache; the captured graph when there is one."""
        if img_u8.shape != self.img.shape:
            raise ValueError(f"image must be {tuple(self.img.shape)} uint8")
        self.img.copy_(img_u8, non_blocking=True)
        if "encode" in self.graphs:
            self.graphs["encode"].replay()
        else:
            self._encode()

    def set_questions(self, questions):
        self.td.set_questions(questions)

    def query(self):
        return self.td.query()

    def decide(self, logits):
        """Per question (pred_yes, argmax or -1, margin); raises first if the frame's fused residual-LayerNorm
        launches reported a timed-out wait (decide reads the logits on the host anyway)."""
        self.vt.check()
        return self.td.decide(logits)

    def frame(self, img_u8):
        """One yes/no frame: encode(img) then query() -> (nq, n_yes + n_no) logits."""
        self.encode(img_u8)
        return self.query()

    # ------------------------------------------------------------------ graphs (md2fast.py:238-256)
    def capture(self):
        """Warm up eagerly (tunes every GEMM shape outside capture), then record encode and query."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self._encode()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._encode()
        torch.cuda.synchronize()
        self.graphs["encode"] = g
        g.replay()  # the prefix the query graph is captured over
        self.td.capture_query()
        return g
