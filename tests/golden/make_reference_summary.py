"""Writes tests/golden/reference_summary.json from the reference's own fixture files.

Run once in the build container, where the reference checkout is mounted (default
/root/reference); the tests read only the JSON it writes. Fixture arrays are read with
numpy.load(allow_pickle=False) and manifest.json as JSON; nothing from the reference is
imported or executed. The fixtures come from the real model (whose weights are absent), so
what is kept is what they fix independently of the weights: shapes, ids, the prompt's row
structure, the generation settings and the reference's recorded codes.
"""
import json
import sys
from pathlib import Path

import numpy as np

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference") / "tests" / "reference"
OUT = Path(__file__).resolve().parent / "reference_summary.json"


def main():
    man = json.loads((REF / "manifest.json").read_text())
    load = lambda n: np.load(REF / n, allow_pickle=False)
    shapes = {p.name: list(np.load(p, allow_pickle=False).shape) for p in sorted(REF.glob("*.npy"))}
    pe, pad, spk = load("prefill_embeds.npy"), load("tts_pad_embed.npy"), load("speaker_embedding.npy").reshape(-1)
    dev = [float(np.abs(pe[r] - pad - spk).max()) for r in range(pe.shape[0])]
    kv = np.load(REF / "prefill_kv.npz", allow_pickle=False)
    out = {
        "source": "reference tests/reference fixtures (Qwen3-TTS-12Hz-0.6B-Base, qwen_tts 0.1.1)",
        "manifest": {k: man[k] for k in ("n_text_ids", "prefill_len", "trailing_len", "greedy_frames", "sampled_frames",
                                         "sampled_samples", "sampled_seed", "sample_rate", "language", "suppress_tokens",
                                         "greedy")},
        "shapes": shapes,
        "prefill_kv": {"n_arrays": len(kv.files), "shape": list(kv[kv.files[0]].shape)},
        "text_ids": load("text_ids.npy").astype(int).tolist(),
        "prefill_position_ids": load("prefill_position_ids.npy").astype(int).tolist(),
        "prefill_mask": load("prefill_mask.npy").astype(int).tolist(),
        "greedy_codes_first2": load("greedy_codes.npy")[:2].astype(int).tolist(),
        "frame0_codes": load("frame0_codes.npy").astype(int).tolist(),
        "prefill_row_minus_pad_minus_speaker_maxabs": dev,
    }
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
