"""Oracle: a CPU restatement of navi-tts's per-frame token loop.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library, the C++
host classes, the `navi_amd` Python plumbing) imports or runs this package.
Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
use it, and only as the checker or the reported CPU baseline.

It restates, from the reference's own sources (cited per function):

* `rng`      - splitmix64 seeding and the PCG32 draw (model/qwen3tts/frame.hip:169-175, 263-296, 581-586, 653-659);
* `sampler`  - modified logits, exact top-k threshold, greedy/multinomial choice (frame.hip:178-296, 413-500);
* `model`    - talker decode step, 16-position code-predictor pass, next-step assembly
               (frame.hip:300-579), prompt assembly and prefill (model/qwen3tts/talker.hip:20-117, 283-399);
* `vocoder`  - the codec decoder (model/qwen3tts/vocoder.hip:20-146, 261-385; kernels.h:72-350).

Precision policy (mirrors the engine's storage points, not its summation order):
f16 weights exactly as stored in the blob, f32 activations and accumulation,
K/V rounded to f16 where the engine stores them to its cache.

Pinning: see tests/test_oracle_*.py. Every function is checked against a golden
vector, a brute force, a textbook known answer or an independent library
implementation (transformers' Qwen3 layer); DESIGN.md lists which check pins
which function and names any function left "parity unpinned".
"""
