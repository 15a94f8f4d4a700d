"""Oracle: a CPU restatement of navi-tts's per-frame token loop.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library, the C++
host classes, the `navi_amd` Python plumbing) imports or runs this package.
Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
use it, and only as the checker or the reported CPU baseline.

It restates, from the reference's own sources (cited per function):

* `rng`       - splitmix64 seeding and the PCG32 draw (model/qwen3tts/frame.hip:169-175, 263-296, 581-586, 653-659);
* `sampler`   - modified logits, exact top-k threshold, greedy/multinomial choice (frame.hip:178-296, 413-500);
* `model`     - talker decode step, 16-position code-predictor pass, next-step assembly
                (frame.hip:300-579), prompt assembly and prefill (model/qwen3tts/talker.hip:20-117, 283-399);
* `navi_read` - the `.navi` reader (docs/navi-format.md; runtime/weights/navi_file.cpp:79-148);
* `vocoder`   - the codec decoder, codes -> PCM (model/qwen3tts/vocoder.hip:20-343, kernels.h:72-242);
* `speaker`   - the speaker encoder's log-mel front end and ECAPA-TDNN (model/qwen3tts/speaker.hip:46-331);
* `csrc/sampler.c` + `csampler` - a second, C restatement of the seeding, the radix k-th-largest
                select and the draw (the same frame.hip lines), used to cross-check `rng`/`sampler`.

Precision policy (mirrors the engine's storage points, not its summation order):
f16 weights exactly as stored in the blob, f32 activations and accumulation,
K/V rounded to f16 where the engine stores them to its cache.

Pinning (tests/test_oracle_*.py, tests/test_blob.py):
* rng: SplitMix64 and PCG32 textbook known answers; Python == C on many seeds;
* sampler: k-th largest three ways (sort, radix select in C, the definition) with ties, -inf and
  signed zeros; fused sum vs libm fmaf; draw Python == C, hand cases, chi-square against the
  softmax; suppression / EOS gate / penalty special cases;
* model: decoder layer vs transformers' Qwen3DecoderLayer (random weights, non-unit norms), with a
  planted-mistake control; prefill == sequential decode; RoPE and RMSNorm closed forms; the
  assembly order; prompt layout vs the reference's fixtures (row counts, speaker row); the text
  projection (fc1 -> SiLU -> fc2) vs transformers' Qwen3OmniMoeTalkerResizeMLP, with
  planted-mistake controls;
* vocoder: SnakeBeta, the residual unit, ConvNeXt and the sliding-window transformer layer vs
  transformers' Qwen3-Omni code2wav modules; causal and transposed convs vs brute-force loops;
  the RVQ front end vs transformers' MimiSplitResidualVectorQuantizer.decode (one semantic
  codebook + the summed acoustic ones, each set through its own 1x1 output projection), with
  planted-mistake controls; causality of the whole decoder;
* speaker: the log-mel vs the reference's own fixture (speaker_mels.npy, first 2 s of
  voice_1.wav); the "same" reflect conv vs torch.nn.Conv1d(padding_mode="reflect");
  weighted statistics vs numpy.average; the whole network on a time-constant mel vs its closed
  form, and on real speech frames vs transformers' ECAPA_TimeDelayNet, each with a planted-mistake
  control;
* code predictor wiring (`Oracle.code_predictor`: which embedding feeds which position, which
  lm_head scores it, the cache positions) vs transformers' Qwen3-Omni talker code predictor
  (random weights, greedy codes and every position's logits), with four planted-mistake controls.
Parity unpinned: none of the functions above. The per-frame composition (`Oracle.frame`) is the
composition of pinned pieces.
"""
