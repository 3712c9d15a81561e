"""Writes the small golden fixtures under tests/golden/ from the oracle (run: python tests/golden/make_golden.py).

The reference ships no vectors for this path, so these are the oracle's own outputs on seeded inputs: they pin the
oracle (and anything checked against it) against silent drift. Each fixture holds inputs and expected outputs:
  vision_block.pt  one tiny pre-LN SigLIP block (D 32, 4 heads), x (2, 11, 32)
  text_prefill.pt  tiny 2-layer text model: prefix + prompt prefill logits and 3 greedy tokens
  ssm.pt           the RG-LRU step (2 heads x 64 channels, 64 tokens) for a first and a later frame
"""
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle.md2_text as ot  # noqa: E402
import oracle.md2_vision as ov  # noqa: E402
import oracle.trecvit as otr  # noqa: E402
import strix_halo_maxx_amd.synth as S  # noqa: E402
import test_oracle as T  # noqa: E402


def main():
    torch.set_num_threads(1)
    w = T._tiny_vision(32, 48, 4)
    x = torch.randn(2, 11, 32, generator=T.gen(21)).to(torch.bfloat16)
    torch.save({"w": w, "x": x, "y": ov.block(w, 0, x, H=4)}, os.path.join(HERE, "vision_block.pt"))

    wt = T._tiny_text(64, 96, 97)
    fr = S.freqs_cis(32, 256)
    img = (torch.randn(13, 64, generator=T.gen(22)) * 0.5).to(torch.bfloat16)
    prompt = torch.randint(0, 97, (6,), generator=T.gen(23))
    m = ot.Text(wt, 64, fr, bos=3, H=2)
    toks, lgs = m.generate(img, prompt, 3)
    torch.save({"w": wt, "img": img, "prompt": prompt, "tokens": torch.tensor(toks), "logits": torch.stack(lgs)},
               os.path.join(HERE, "text_prefill.pt"))

    d = T._ssm_case(seed=24)
    out = {"inputs": d}
    for first in (True, False):
        z, h = T._run_ssm(d, first)
        out[f"z_{int(first)}"], out[f"h_{int(first)}"] = z, h
    torch.save(out, os.path.join(HERE, "ssm.pt"))


if __name__ == "__main__":
    main()
