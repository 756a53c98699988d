"""Writes tests/golden/tiny_greedy.npz.

The fixture holds the last-row logits and greedy tokens of a tiny akasha
model (ModelConfig::new(97, 64, 2, 2, 48), synthetic weights seed 21) for a
12-token prompt followed by 8 greedy steps.  Expected values come from a
float64 numpy forward that recomputes the whole prefix at every step, so the
fixture shares no code with the C oracle or the HIP library.

Run from the repository root: python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE.parent))

import __graft_entry__ as entry  # noqa: E402
from test_oracle import _forward64  # noqa: E402


def main():
    pkg = entry.load_package()
    cfg_args = (97, 64, 2, 2, 48)
    cfg = pkg.ModelConfig.new(*cfg_args)
    seed = 21
    w = pkg.synthetic_weights(cfg, seed=seed)
    prompt = np.random.default_rng(22).integers(0, 97, 12).astype(np.uint32)
    seq = list(prompt)
    logits, tokens = [], []
    for _ in range(8):
        lg = _forward64(cfg, w, np.array(seq))
        t = int(np.argmax(lg))
        srt = np.sort(lg)
        assert srt[-1] - srt[-2] > 1e-4, "near-tie: pick another seed"
        logits.append(lg.astype(np.float32))
        tokens.append(t)
        seq.append(t)
    np.savez_compressed(HERE / "tiny_greedy.npz", cfg=np.array(cfg_args), seed=seed,
                        max_ctx=48, prompt=prompt, logits=np.stack(logits),
                        tokens=np.array(tokens, np.uint32))
    print("tokens", tokens)


if __name__ == "__main__":
    main()
