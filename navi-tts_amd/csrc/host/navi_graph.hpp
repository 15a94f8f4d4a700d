// The reference's C++ request interface over this library's C ABI: navi::qwen3tts::Graph with
// the signatures of model/qwen3tts/graph.h:23-79, so the HTTP server's paths
// (runtime/server/server.cpp:401-437 speak / speak_stream, 770-788 warm_up) call it as they call
// the reference. Header-only (C++20 for std::span, as the reference): the shared library keeps
// exporting plain C.
//
// What the host keeps from the reference: the tokenizer (plugged in as `tokenize`, text -> ids;
// SynthRequest::text is wrapped in the assistant turn as graph.cpp:59 does) and the weight
// loading (the handles arrive created). Semantics kept: PCM per vocoder batch on the calling
// thread; an exception thrown by on_pcm stops the request before another frame runs and leaves
// synth (the server's "client stopped reading"); a failed frame throws navi::Error.
#pragma once

#include "navi_amd.h"

#include <chrono>
#include <cstdint>
#include <exception>
#include <functional>
#include <map>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

namespace navi {

// runtime/common/error.h:10-14
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

namespace qwen3tts {

constexpr int STREAM_FIRST_BATCH = 4;   // graph.h:29-30: frames in the first vocoder call, then
constexpr int STREAM_BATCH = 16;        // per call; batching never changes the PCM

// frame.h:24-31 defaults (the model's generation_config.json)
struct Sampling {
    float temperature = 0.9f;
    int top_k = 50;
    float repetition_penalty = 1.05f;
    float cp_temperature = 0.9f;
    int cp_top_k = 50;
    int min_frames = 2;
};

struct SynthRequest {                    // graph.h:32-41 (+ ids for callers that tokenize themselves)
    std::string text;
    std::string language = "english";
    std::span<const float> speaker;      // [hidden]
    std::uint64_t seed = 0;
    int max_frames = 600;
    Sampling sampling;
    int vocoder_batch = 0;               // 0: the vocoder's max chunk
    int first_batch = 0;                 // 0: vocoder_batch
    std::vector<std::int32_t> ids;       // used as given when non-empty (text ignored)
};

struct SynthStats {                      // graph.h:43-48
    int n_tokens = 0, n_frames = 0;
    bool hit_cap = false, eos = false;
    double tokenize_ms = 0, prefill_ms = 0, frames_ms = 0, vocoder_ms = 0, total_ms = 0, ttfa_ms = 0;
    double audio_s = 0, rtf = 0;
};

class Graph {
public:
    using Tokenize = std::function<std::vector<std::int32_t>(const std::string &)>;

    // Borrows the handles (the caller destroys them after the Graph). languages: name -> codec
    // language id (the .navi's talker.language.<name> keys); speaker may be null.
    Graph(navi_talker *talker, navi_frame *frame, navi_vocoder *vocoder, navi_speaker *speaker,
          std::map<std::string, int> languages, Tokenize tokenize = {})
        : t_(talker), f_(frame), v_(vocoder), s_(speaker), languages_(std::move(languages)), tokenize_(std::move(tokenize)) {}

    // graph.h:64-65
    std::vector<float> embed_speaker(std::span<const float> wav_24k) {
        if (!s_) throw Error("graph: no speaker encoder");
        std::vector<float> out(static_cast<size_t>(navi_speaker_dim(s_)));
        char err[256] = {};
        check(navi_speaker_embed(s_, wav_24k.data(), static_cast<int64_t>(wav_24k.size()), out.data(), err, sizeof err), err);
        return out;
    }

    // graph.h:67-69: every vocoder batch's PCM goes to on_pcm as it is produced
    SynthStats synth(const SynthRequest &req, const std::function<void(std::span<const float>)> &on_pcm) {
        std::vector<std::int32_t> ids = req.ids;
        double tokenize_ms = 0;
        if (ids.empty()) {
            if (!tokenize_) throw Error("graph: no tokenizer for a text request");
            const auto t0 = std::chrono::steady_clock::now();
            ids = tokenize_("<|im_start|>assistant\n" + req.text + "<|im_end|>\n<|im_start|>assistant\n");
            tokenize_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        }
        if (static_cast<int>(ids.size()) - 8 < 1) throw Error("empty text");
        int lang = -1;
        if (!req.language.empty() && req.language != "auto") {
            const auto it = languages_.find(req.language);
            if (it == languages_.end()) throw Error("unknown language '" + req.language + "'");
            lang = it->second;
        }
        if (req.speaker.size() != 1024) throw Error("graph: speaker embedding must have 1024 values");
        navi_synth_request r{};
        r.ids = ids.data();
        r.n_ids = static_cast<int32_t>(ids.size());
        r.language_id = lang;
        r.speaker = req.speaker.data();
        r.seed = req.seed;
        r.max_frames = req.max_frames;
        r.sampling = navi_sampling{req.sampling.temperature, req.sampling.top_k, req.sampling.repetition_penalty,
                                   req.sampling.cp_temperature, req.sampling.cp_top_k, req.sampling.min_frames};
        r.vocoder_batch = req.vocoder_batch;
        r.first_batch = req.first_batch;
        struct Ctx {
            const std::function<void(std::span<const float>)> *fn;
            std::exception_ptr thrown;
        } ctx{&on_pcm, nullptr};
        auto trampoline = [](const float *pcm, int32_t n, void *user) -> int32_t {
            auto *c = static_cast<Ctx *>(user);
            try {
                (*c->fn)(std::span<const float>(pcm, static_cast<size_t>(n)));
                return 0;
            } catch (...) {
                c->thrown = std::current_exception();
                return 1;
            }
        };
        navi_synth_stats st{};
        char err[256] = {};
        const navi_status s = navi_synth(t_, f_, v_, &r, trampoline, &ctx, &st, err, sizeof err);
        if (ctx.thrown) std::rethrow_exception(ctx.thrown);
        check(s, err);
        SynthStats out;
        out.n_tokens = st.n_tokens;
        out.n_frames = st.n_frames;
        out.hit_cap = st.hit_cap != 0;
        out.eos = st.eos != 0;
        out.tokenize_ms = tokenize_ms;
        out.prefill_ms = st.prefill_ms + tokenize_ms;   // graph.h:46: prefill_ms includes tokenize_ms
        out.frames_ms = st.frames_ms;
        out.vocoder_ms = st.vocoder_ms;
        out.total_ms = st.total_ms + tokenize_ms;
        out.ttfa_ms = st.ttfa_ms + tokenize_ms;
        out.audio_s = st.audio_s;
        out.rtf = st.rtf;
        return out;
    }

    // graph.h:71-72: the whole utterance into one buffer
    SynthStats synth(const SynthRequest &req, std::vector<float> &pcm) {
        pcm.clear();
        return synth(req, [&](std::span<const float> chunk) { pcm.insert(pcm.end(), chunk.begin(), chunk.end()); });
    }

private:
    static void check(navi_status s, const char *err) {
        if (s != NAVI_OK) throw Error(err && *err ? err : "navi: call failed");
    }

    navi_talker *t_;
    navi_frame *f_;
    navi_vocoder *v_;
    navi_speaker *s_;
    std::map<std::string, int> languages_;
    Tokenize tokenize_;
};

} // namespace qwen3tts
} // namespace navi
