"""Writes the golden fixtures of this directory: for each seeded workload, the
oracle's outputs on its first 8 rows (batch 0), after checking every id
against the independent Python restatement (tests/np_ref.py) where that
restatement covers the variant; plus one indextts beam-sample step.  Inputs
are not stored: they are regenerated from their seeds (talechime_amd.synth),
and each fixture records the sha256 of the input bytes it was made from.
MANIFEST.sha256 lists the fixtures' own hashes.

    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from talechime_amd import synth  # noqa: E402
from tests import np_ref  # noqa: E402

ROWS = 8
CAP = 64


def input_hash(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def params(w):
    return O.make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                         min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)


def cross_check(w, b, o):
    """The ids of the rows np_ref restates, against the oracle's."""
    for r in range(ROWS):
        h = b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]]
        x = b.logits_f32[r]
        if w.variant == O.QWEN:
            if o["flags"][r] & 1:
                continue
            want = np_ref.qwen_row(x, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                                   seen_ids=h, u=b.uniforms[r])
        elif w.variant == O.INDEXTTS:
            want = np_ref.indextts_row(x, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                                       penalty=w.penalty, hist=h, u=b.uniforms[r])
        elif w.variant == O.COSY_RAS:
            want = np_ref.cosy_row(x, top_p=w.top_p, top_k=w.top_k, win=w.ras_win, tau=w.ras_tau, hist=h,
                                   u0=b.uniforms[2 * r], u1=b.uniforms[2 * r + 1])[0]
        else:
            continue
        assert int(o["ids"][r]) == int(want), (w.name, r, int(o["ids"][r]), want)


def main():
    names = []
    for name, w in synth.WORKLOADS.items():
        b = synth.make_batch(w, rows=ROWS)
        o = O.sample(params(w), b.logits_f32, b.hist_off, b.hist_ids, b.uniforms, cap=CAP)
        if w.variant != O.QWEN or w.vocab <= 16384:
            cross_check(w, b, o)
        fn = f"{name}.npz"
        np.savez_compressed(os.path.join(HERE, fn), ids=o["ids"], status=o["status"], flags=o["flags"],
                            topk_count=o["topk_count"], topk_ids=o["topk_ids"], keep_count=o["keep_count"],
                            keep_ids=o["keep_ids"], keep_probs=o["keep_probs"], norm=o["norm"],
                            input_sha256=np.array(input_hash(b.logits_f32, b.hist_off, b.hist_ids, b.uniforms)))
        names.append(fn)
    # one beam-sample step: 2 elements x 3 beams of the indextts rows (later step)
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    bb = synth.make_beam_batch(w, 2, 3)
    p = O.make_params(O.INDEXTTS, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                      min_keep=w.min_keep)
    ob = O.idx_beam_step(p, bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, 3, bb.uniforms, 6)
    for bi in range(2):
        rows = [bb.logits[bi * 3 + j] for j in range(3)]
        hists = [bb.hist_ids[bb.hist_off[bi * 3 + j]:bb.hist_off[bi * 3 + j + 1]] for j in range(3)]
        want = np_ref.indextts_beam_step(rows, hists, bb.beam_scores[bi * 3:bi * 3 + 3], 3,
                                         bb.uniforms[bi * 6:bi * 6 + 6], 6, temperature=w.temperature,
                                         top_k=w.top_k, top_p=w.top_p, penalty=w.penalty, min_keep=w.min_keep)
        assert [(float(s), int(f)) for s, f in zip(ob["scores"][bi], ob["flat"][bi])] == want
    fn = "indextts-beam-2x3x8194.npz"
    np.savez_compressed(os.path.join(HERE, fn), flat=ob["flat"], scores=ob["scores"], status=ob["status"],
                        input_sha256=np.array(input_hash(bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores,
                                                         bb.uniforms)))
    names.append(fn)
    with open(os.path.join(HERE, "MANIFEST.sha256"), "w") as f:
        for fn in sorted(names):
            f.write(hashlib.sha256(open(os.path.join(HERE, fn), "rb").read()).hexdigest() + "  " + fn + "\n")
    print(json.dumps({"fixtures": sorted(names)}))


if __name__ == "__main__":
    main()
