"""Pins the oracle's prompt assembly and prefill (Oracle.build_prompt / Oracle.prefill).

The reference's fixtures (summarised in tests/golden/reference_summary.json by
tests/golden/make_reference_summary.py) come from the real weights, which are absent; what
they fix independently of the weights is checked here: the 25 fixture ids give a 10-row
prefill and 17 trailing rows, position ids 0..9, an all-ones mask, and row 7 - and only
row 7 - is tts_pad + speaker. The prefill's last row is checked against the same rows run
as sequential decode steps.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_summary.json").read_text())


@pytest.fixture(scope="module")
def ora(small_blob):
    from oracle.model import Oracle
    return Oracle(small_blob)


def test_fixture_summary_is_self_consistent():
    m = GOLDEN["manifest"]
    assert len(GOLDEN["text_ids"]) == m["n_text_ids"] == 25
    assert GOLDEN["shapes"]["prefill_embeds.npy"] == [m["prefill_len"], 1024]
    assert GOLDEN["shapes"]["trailing_text.npy"] == [m["trailing_len"], 1024]
    assert GOLDEN["prefill_position_ids"] == [list(range(10))] * 3
    assert GOLDEN["prefill_mask"] == [1] * 10
    assert GOLDEN["frame0_codes"] == GOLDEN["greedy_codes_first2"][0]


def test_prompt_shape_matches_reference_fixture(ora):
    rng = np.random.default_rng(0)
    spk = rng.standard_normal(1024).astype(np.float32)
    pre, trail, pad = ora.build_prompt(GOLDEN["text_ids"], GOLDEN["manifest"]["language"], spk)
    assert pre.shape == tuple(GOLDEN["shapes"]["prefill_embeds.npy"])
    assert trail.shape == tuple(GOLDEN["shapes"]["trailing_text.npy"])
    assert pad.shape == tuple(GOLDEN["shapes"]["tts_pad_embed.npy"])


def test_speaker_row_position_matches_reference_fixture(ora):
    ref_dev = np.asarray(GOLDEN["prefill_row_minus_pad_minus_speaker_maxabs"])
    ref_rows = np.flatnonzero(ref_dev < 1e-6)
    assert ref_rows.tolist() == [7]
    spk = np.random.default_rng(1).standard_normal(1024).astype(np.float32)
    pre, _, pad = ora.build_prompt(GOLDEN["text_ids"], "english", spk)
    dev = np.array([np.abs(pre[r] - pad - spk).max() for r in range(pre.shape[0])])
    assert np.flatnonzero(dev < 1e-6).tolist() == ref_rows.tolist()


def test_prompt_rows_follow_the_text(ora):
    """Changing one body token changes exactly the rows that carry it: row 9 holds text[0]
    (plus codec_bos); trailing row j holds text[j + 1]; the last trailing row is tts_eos."""
    ids = list(GOLDEN["text_ids"])
    spk = np.zeros(1024, np.float32)
    pre, trail, _ = ora.build_prompt(ids, "english", spk)
    ids2 = ids.copy()
    ids2[3] = 1000                       # text[0]
    ids2[8] = 2000                       # text[5] -> trailing row 4
    pre2, trail2, _ = ora.build_prompt(ids2, "english", spk)
    assert [r for r in range(10) if not np.array_equal(pre[r], pre2[r])] == [9]
    assert [r for r in range(17) if not np.array_equal(trail[r], trail2[r])] == [4]


def test_auto_language_drops_the_language_row(ora):
    spk = np.zeros(1024, np.float32)
    pre, trail, _ = ora.build_prompt(GOLDEN["text_ids"], "auto", spk)
    assert pre.shape[0] == 9 and trail.shape[0] == 17


def test_prefill_last_row_equals_sequential_steps(ora):
    rng = np.random.default_rng(2)
    pre, _, _ = ora.build_prompt(GOLDEN["text_ids"], "english", rng.standard_normal(1024).astype(np.float32))
    kv_a, kv_b = ora.new_kv(16), ora.new_kv(16)
    h_a, lg_a = ora.prefill(pre, kv_a)
    for t in range(pre.shape[0]):
        h_b, lg_b = ora.talker_step(pre[t], kv_b, t)
    assert np.allclose(h_a, h_b, atol=2e-4) and np.allclose(lg_a, lg_b, atol=2e-4)
    for l in range(ora.tp.n_layer):
        for a, b in zip(kv_a[l], kv_b[l]):
            # layer > 0 inputs already differ by accumulation order: a few f16 ulps
            assert torch.allclose(a[:10], b[:10], rtol=4e-3, atol=1e-3)
