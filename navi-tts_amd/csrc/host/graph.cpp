// One request end to end over the C ABI: prompt -> prefill -> frames -> vocoder batches
// (Graph::synth, model/qwen3tts/graph.cpp:52-111), host code only.
//
// The request arrives tokenized (the tokenizer is not part of this library). Streaming
// follows the reference: the vocoder runs as soon as first_batch frames (then vocoder_batch
// frames) are pending, so time to first audio = prompt + prefill + first_batch frames + one
// vocoder call; batching never changes the PCM (the vocoder is causal with carried state).
#include "navi_amd.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdarg>
#include <vector>

namespace {

using clk = std::chrono::steady_clock;

double ms_since(clk::time_point a) { return std::chrono::duration<double, std::milli>(clk::now() - a).count(); }

void put_err(char *err, size_t errlen, const char *fmt, ...) {
    if (!err || !errlen) return;
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

} // namespace

extern "C" navi_status navi_synth(navi_talker *t, navi_frame *f, navi_vocoder *v, const navi_synth_request *req,
                                  navi_pcm_callback on_pcm, void *user, navi_synth_stats *stats, char *err, size_t errlen) {
    if (!t || !f || !v || !req || !stats) {
        put_err(err, errlen, "synth: null argument");
        return NAVI_ERR_INVALID;
    }
    *stats = navi_synth_stats{};
    const auto t0 = clk::now();
    navi_prompt pr{};
    navi_status st;
    if (req->d_prefill) {
        if (!req->d_trailing || !req->d_tts_pad || req->n_prefill < 1 || req->n_trailing < 0) {
            put_err(err, errlen, "synth: incomplete prompt rows");
            return NAVI_ERR_INVALID;
        }
        pr.prefill = req->d_prefill;
        pr.trailing = req->d_trailing;
        pr.tts_pad = req->d_tts_pad;
        pr.n_prefill = req->n_prefill;
        pr.n_trailing = req->n_trailing;
        stats->n_tokens = req->n_trailing;
    } else {
        if ((st = navi_talker_build_prompt(t, req->ids, req->n_ids, req->language_id, req->speaker, &pr, err, errlen)) != NAVI_OK)
            return st;
        stats->n_tokens = req->n_ids - 8;
    }
    if ((st = navi_talker_prefill(t, pr.prefill, pr.n_prefill, err, errlen)) != NAVI_OK) return st;
    stats->prefill_ms = ms_since(t0);

    navi_kv_view kv{};
    if ((st = navi_talker_kv(t, &kv, nullptr)) != NAVI_OK) return st;
    if ((st = navi_frame_reset(f)) != NAVI_OK || (st = navi_vocoder_reset(v)) != NAVI_OK) {
        put_err(err, errlen, "synth: reset failed");
        return st;
    }
    const int spf = navi_vocoder_samples_per_frame(v), cmax = navi_vocoder_max_chunk_frames(v);
    const int batch = req->vocoder_batch > 0 ? std::min(req->vocoder_batch, cmax) : cmax;
    const int first = req->first_batch > 0 ? std::min(req->first_batch, batch) : batch;
    const size_t H = 1024;
    std::vector<int32_t> codes;
    std::vector<float> pcm;
    int pending = 0;
    bool first_audio = true;
    auto flush = [&](bool final) -> navi_status {
        if (pending == 0 || (!final && pending < (first_audio ? first : batch))) return NAVI_OK;
        const auto tv = clk::now();
        pcm.resize(static_cast<size_t>(pending) * spf);
        const navi_status s = navi_vocoder_decode(v, codes.data() + codes.size() - static_cast<size_t>(pending) * 16, pending,
                                                  pcm.data(), err, errlen);
        if (s != NAVI_OK) return s;
        stats->vocoder_ms += ms_since(tv);
        pending = 0;
        if (first_audio) {
            stats->ttfa_ms = ms_since(t0);
            first_audio = false;
        }
        if (on_pcm && on_pcm(pcm.data(), static_cast<int32_t>(pcm.size()), user) != 0) {
            put_err(err, errlen, "synth: stopped by the PCM consumer after %d frames", stats->n_frames);
            return NAVI_ERR_CANCELLED;
        }
        return NAVI_OK;
    };
    // Frames run in on-device loops of exactly the vocoder's batch sizes (first batch, then
    // vocoder_batch): no host round trip between the frames of a batch, the same PCM batches the
    // reference's per-frame loop produces.
    std::vector<int32_t> batch_codes(static_cast<size_t>(std::max(batch, first)) * 16);
    for (int i = 0; i < req->max_frames && !stats->eos;) {
        // the flush below empties pending; a loop never crosses the end of the KV cache, so a full
        // cache fails at the frame that hits it, after the frames before it were delivered
        const int fit = kv.max_pos - (pr.n_prefill - 1 + i);
        const int want = std::max(1, std::min({i == 0 ? first : batch, req->max_frames - i, fit}));
        const int n_trail_left = std::max(0, pr.n_trailing - i);
        int32_t done = 0, eos = 0;
        double us = 0.0;
        // global frame g >= 1 runs at n_prefill + g - 1; frame 0 is run_first from the prefill's outputs
        const navi_status s = navi_frame_run_many(f, &kv, pr.n_prefill - 1 + i, i == 0 ? 1 : 0,
                                                  navi_talker_hidden(t), navi_talker_logits(t),
                                                  n_trail_left ? pr.trailing + static_cast<size_t>(i) * H : nullptr, n_trail_left,
                                                  pr.tts_pad, &req->sampling, req->seed, i, want, batch_codes.data(), &done, &eos,
                                                  &us, err, errlen);
        if (s != NAVI_OK) {
            if (err && errlen) {
                char tmp[256];
                std::snprintf(tmp, sizeof tmp, "%s", err);
                put_err(err, errlen, "frame %d: %s", i + done, tmp);
            }
            return s;
        }
        stats->frames_ms += us / 1000.0;
        const int kept = eos ? done - 1 : done;
        codes.insert(codes.end(), batch_codes.begin(), batch_codes.begin() + static_cast<size_t>(kept) * 16);
        stats->n_frames += kept;
        pending += kept;
        i += done;
        if (eos) {
            stats->eos = 1;
            break;
        }
        if ((st = flush(false)) != NAVI_OK) {
            stats->total_ms = ms_since(t0);
            return st;
        }
    }
    stats->hit_cap = !stats->eos;
    st = flush(true);
    stats->total_ms = ms_since(t0);
    stats->audio_s = static_cast<double>(stats->n_frames) * spf / 24000.0;
    stats->rtf = stats->audio_s > 0 ? stats->total_ms / 1000.0 / stats->audio_s : 0.0;
    return st;
}
