"""The whole moondream2 yes/no frame (strix_halo_maxx_amd.md2frame.FastMD2: vision tower -> projection -> 730-token
prefix prefill, then the batched yes/no query; md2fast.py:147-160, 201-212, 238-265) against the oracle chain
(oracle.md2_vision.tower(project=True) -> oracle.md2_text.Text.encode -> query) on 2 vision and 2 text layers.
Tolerances: yes/no logits rel-L2 <= 2e-2 per question (the vision end-to-end bound carried through the text layers);
decide() agrees with the oracle wherever the oracle's margin exceeds twice the largest logit difference (logsumexp
is 1-Lipschitz in the max norm, so only such a margin can change sign); the captured encode + query graphs replay the
eager frame bit for bit and follow a new image between replays."""
import pytest
import torch

import oracle.md2_text as ot
import oracle.md2_vision as ov
import strix_halo_maxx_amd.md2frame as mf
import strix_halo_maxx_amd.synth as S

pytestmark = pytest.mark.gpu
YES, NO = [11, 222, 3333, 44444], [55, 666, 7777, 50000]


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _oracle_frame(vw, tw, img, qs, L):
    emb = ov.tower(vw, img, project=True)[0]
    ora = ot.Text(tw, 1024, S.freqs_cis(32, 2048))
    ora.encode(emb)
    return ora.query(qs, L, YES + NO)


def test_frame_two_layers_vs_oracle_chain_and_graphs(dev):
    vw = S.vision_weights(0, layers=2, proj=True)
    tw = S.text_weights(0, layers=2)
    imgs = S.images_u8(21, 2)
    qs = [S.prompt_ids(50 + n, n).tolist() for n in (9, 32)]
    f = mf.FastMD2(vw, tw, device=dev, nq=2, L=32, yes_ids=YES, no_ids=NO)
    f.set_questions(qs)
    eager = []
    for i in range(2):
        lg = f.frame(imgs[i].to(dev)).cpu().clone()
        eager.append(lg)
        ref = _oracle_frame(vw, tw, imgs[i:i + 1], qs, 32)
        for b in range(2):
            r = rel(lg[b], ref[b])
            print(f"image {i} question {b}: yes/no logits rel-L2 {r:.2e}", flush=True)
            assert r <= 2e-2
            emax = (lg[b].float() - ref[b].float()).abs().max().item()
            p, _, m = f.decide(lg[b])[0]
            rp, rm = ot.Text.decide(ref[b], len(YES))
            assert abs(m - rm) <= 2 * emax + 1e-5
            if abs(rm) > 2 * emax:
                assert p == rp
    f.capture()
    for _ in range(2):
        for i in (1, 0):
            lg = f.frame(imgs[i].to(dev)).cpu()
            assert torch.equal(lg, eager[i]), i


def test_frame_rejects_a_tower_without_projection(dev):
    with pytest.raises(ValueError):
        mf.FastMD2(S.vision_weights(0, layers=1), S.text_weights(0, layers=1), device=dev)
