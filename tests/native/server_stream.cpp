// The HTTP server's streaming path (runtime/server/server.cpp:401-495, 770-788) driven through
// navi_graph.hpp: a test harness, built as a shared library that tests/test_server_stream_gpu.py
// loads with ctypes and hands the created talker / frame / vocoder / speaker handles.
//
// What the server does with a Graph, restated here: one worker thread owns the GPU and runs
// Graph::synth; its on_pcm converts each vocoder batch to s16 and pushes it into a bounded
// queue, throwing "client stopped reading" when the push fails; the consumer waits for the
// first batch (its arrival is the time to first audio), then drains the queue or aborts it.
// The scenarios report what they saw as one JSON object; the Python test asserts on it.
#include "navi_graph.hpp"

#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

using navi::qwen3tts::Graph;
using navi::qwen3tts::SynthRequest;
using navi::qwen3tts::SynthStats;

// runtime/audio/wav.cpp:13-22: clamp to [-1, 1], scale by 32767, round to nearest
std::vector<int16_t> to_s16(std::span<const float> pcm) {
    std::vector<int16_t> out(pcm.size());
    for (size_t i = 0; i < pcm.size(); ++i) out[i] = static_cast<int16_t>(std::lrintf(std::fmax(-1.f, std::fmin(1.f, pcm[i])) * 32767.f));
    return out;
}

// The server's bounded hand-off between the worker and the HTTP writer (server.cpp:100-150):
// a producer that finds the queue aborted (or full past the timeout) is told to stop.
class ChunkQueue {
public:
    explicit ChunkQueue(size_t capacity = 16, std::chrono::milliseconds push_timeout = std::chrono::seconds(10))
        : cap_(capacity), timeout_(push_timeout) {}

    bool push(std::vector<int16_t> chunk) {
        std::unique_lock<std::mutex> l(m_);
        if (!cv_.wait_for(l, timeout_, [&] { return aborted_ || q_.size() < cap_; })) aborted_ = true;
        if (aborted_) return false;
        q_.push_back(std::move(chunk));
        ++pushed_;
        cv_.notify_all();
        return true;
    }
    void finish(std::string error) {
        std::lock_guard<std::mutex> l(m_);
        done_ = true;
        error_ = std::move(error);
        cv_.notify_all();
    }
    bool pop(std::vector<int16_t> &chunk) {
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [&] { return done_ || !q_.empty(); });
        if (q_.empty()) return false;
        chunk = std::move(q_.front());
        q_.pop_front();
        cv_.notify_all();
        return true;
    }
    // true: audio is coming; done_at_first: whether the producer had already finished
    bool wait_first(bool &done_at_first) {
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [&] { return done_ || !q_.empty(); });
        done_at_first = done_;
        return !q_.empty();
    }
    void abort() {
        std::lock_guard<std::mutex> l(m_);
        aborted_ = true;
        q_.clear();
        cv_.notify_all();
    }
    std::string error() const {
        std::lock_guard<std::mutex> l(m_);
        return error_;
    }
    int pushed() const {
        std::lock_guard<std::mutex> l(m_);
        return pushed_;
    }

private:
    mutable std::mutex m_;
    std::condition_variable cv_;
    std::deque<std::vector<int16_t>> q_;
    size_t cap_;
    std::chrono::milliseconds timeout_;
    bool done_ = false, aborted_ = false;
    int pushed_ = 0;
    std::string error_;
};

struct Report {
    std::string s = "{";
    void add(const char *k, double v) { item(k, std::to_string(v)); }
    void add(const char *k, long long v) { item(k, std::to_string(v)); }
    void add(const char *k, int v) { item(k, std::to_string(v)); }
    void add(const char *k, bool v) { item(k, v ? "true" : "false"); }
    void add(const char *k, const std::string &v) {
        std::string e;
        for (char c : v) e += (c == '"' || c == '\\') ? std::string("\\") + c : std::string(1, c);
        item(k, "\"" + e + "\"");
    }
    void add(const char *k, const std::vector<int> &v) {
        std::string a = "[";
        for (size_t i = 0; i < v.size(); ++i) a += (i ? "," : "") + std::to_string(v[i]);
        item(k, a + "]");
    }
    void item(const char *k, const std::string &v) { s += (s.size() > 1 ? "," : "") + std::string("\"") + k + "\":" + v; }
    int put(char *out, size_t n) {
        s += "}";
        std::snprintf(out, n, "%s", s.c_str());
        return s.size() < n ? 0 : 1;
    }
};

// speak_stream: the worker runs synth into the queue; returns the stats and the error text.
void stream_worker(Graph &g, const SynthRequest &sr, ChunkQueue &q, SynthStats &st, std::string &error) {
    try {
        st = g.synth(sr, [&](std::span<const float> pcm) {
            if (!q.push(to_s16(pcm))) throw navi::Error("client stopped reading");
        });
    } catch (const std::exception &e) {
        error = e.what();
    }
    q.finish(error);
}

} // namespace

extern "C" {

// Scenario "stream then one-shot then abort then one-shot": the streamed s16 equals the one-shot
// request's s16 sample for sample; a consumer that aborts at the first batch stops the request
// (the worker's next push fails, synth leaves with the consumer's exception, no further frame
// runs); the same Graph then serves the next request identically.
int navi_test_server_stream(navi_talker *t, navi_frame *f, navi_vocoder *v, navi_speaker *s, int32_t english_id,
                            const int32_t *ids, int32_t n_ids, uint64_t seed, int32_t max_frames, char *out, size_t out_len) {
    Report rep;
    try {
        Graph g(t, f, v, s, {{"english", english_id}});
        // warm_up (server.cpp:770-788): a speaker from 2 s of silence, then a short request
        std::vector<float> speaker(1024, 0.f);
        if (s) {
            const std::vector<float> silence(48000, 0.f);
            speaker = g.embed_speaker(silence);
            double norm = 0;
            for (float x : speaker) norm += static_cast<double>(x) * x;
            rep.add("warmup_speaker_norm", std::sqrt(norm));
        } else {
            for (size_t i = 0; i < speaker.size(); ++i) speaker[i] = std::sin(0.37f * static_cast<float>(i));
        }
        SynthRequest sr;
        sr.ids.assign(ids, ids + n_ids);
        sr.speaker = speaker;
        sr.seed = seed;
        sr.max_frames = max_frames;
        sr.sampling.min_frames = max_frames;          // no early EOS: a fixed number of batches
        sr.first_batch = navi::qwen3tts::STREAM_FIRST_BATCH;
        sr.vocoder_batch = navi::qwen3tts::STREAM_BATCH;
        {
            std::vector<float> warm;
            SynthRequest w = sr;
            w.max_frames = 16;
            w.sampling.min_frames = 2;
            const SynthStats ws = g.synth(w, warm);
            rep.add("warmup_frames", ws.n_frames);
        }

        // 1. streamed
        std::vector<int16_t> streamed;
        std::vector<int> sizes;
        bool done_at_first = true;
        SynthStats st1;
        std::string err1;
        {
            ChunkQueue q;
            std::thread worker([&] { stream_worker(g, sr, q, st1, err1); });
            const bool audio = q.wait_first(done_at_first);
            std::vector<int16_t> c;
            while (audio && q.pop(c)) {
                sizes.push_back(static_cast<int>(c.size()));
                streamed.insert(streamed.end(), c.begin(), c.end());
            }
            worker.join();
        }
        rep.add("stream_error", err1);
        rep.add("stream_frames", st1.n_frames);
        rep.add("stream_sizes", sizes);
        rep.add("stream_first_before_done", !done_at_first);
        rep.add("stream_ttfa_ms", st1.ttfa_ms);
        rep.add("stream_total_ms", st1.total_ms);

        // 2. one shot (speak: synth into a buffer, then to_s16)
        std::vector<float> pcm;
        const SynthStats st2 = g.synth(sr, pcm);
        const std::vector<int16_t> one = to_s16(pcm);
        rep.add("oneshot_frames", st2.n_frames);
        rep.add("stream_equals_oneshot", one == streamed);

        // 3. the client goes away at the first batch
        SynthStats st3;
        std::string err3;
        int pushed = 0;
        double abort_ms = 0;
        {
            ChunkQueue q(1);                              // one slot: the second push waits for the abort
            const auto t0 = std::chrono::steady_clock::now();
            std::thread worker([&] { stream_worker(g, sr, q, st3, err3); });
            bool d = false;
            q.wait_first(d);
            q.abort();
            worker.join();
            abort_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            pushed = q.pushed();
        }
        rep.add("abort_error", err3);
        rep.add("abort_pushed", pushed);
        rep.add("abort_wall_ms", abort_ms);

        // 4. the next request on the same Graph
        std::vector<float> pcm4;
        g.synth(sr, pcm4);
        rep.add("after_abort_equals_oneshot", to_s16(pcm4) == one);

        // 5. a failing request reports through the exception, as the reference's fail()
        SynthRequest bad = sr;
        bad.language = "klingon";
        std::string err5;
        try {
            g.synth(bad, pcm4);
        } catch (const navi::Error &e) {
            err5 = e.what();
        }
        rep.add("bad_language_error", err5);
    } catch (const std::exception &e) {
        rep.add("fatal", std::string(e.what()));
    }
    return rep.put(out, out_len);
}

// Scenario "one request as the server streams it": the worker runs synth with the given sampling
// into the bounded queue, the consumer drains it; the s16 samples it received (in order) and the
// batch sizes go back to the caller for a comparison with the oracle's request. Returns 0, or 1
// with the error text in err.
int navi_test_server_stream_request(navi_talker *t, navi_frame *f, navi_vocoder *v, int32_t english_id,
                                    const int32_t *ids, int32_t n_ids, const float *speaker, uint64_t seed,
                                    int32_t max_frames, float temperature, float cp_temperature, int16_t *pcm_out,
                                    int64_t pcm_cap, int64_t *n_pcm, int32_t *sizes_out, int32_t max_sizes,
                                    int32_t *n_sizes, char *err, size_t errlen) {
    try {
        Graph g(t, f, v, nullptr, {{"english", english_id}});
        SynthRequest sr;
        sr.ids.assign(ids, ids + n_ids);
        sr.speaker = std::span<const float>(speaker, 1024);
        sr.seed = seed;
        sr.max_frames = max_frames;
        sr.sampling.temperature = temperature;
        sr.sampling.cp_temperature = cp_temperature;
        sr.sampling.min_frames = max_frames;
        sr.first_batch = navi::qwen3tts::STREAM_FIRST_BATCH;
        sr.vocoder_batch = navi::qwen3tts::STREAM_BATCH;
        ChunkQueue q;
        SynthStats st;
        std::string error;
        std::thread worker([&] { stream_worker(g, sr, q, st, error); });
        bool done_at_first = true;
        const bool audio = q.wait_first(done_at_first);
        std::vector<int16_t> c;
        int64_t n = 0;
        int32_t k = 0;
        bool overflow = false;
        while (audio && q.pop(c)) {
            if (n + static_cast<int64_t>(c.size()) > pcm_cap || k >= max_sizes) {
                q.abort();
                overflow = true;
                break;
            }
            std::copy(c.begin(), c.end(), pcm_out + n);
            n += static_cast<int64_t>(c.size());
            sizes_out[k++] = static_cast<int32_t>(c.size());
        }
        worker.join();
        *n_pcm = n;
        *n_sizes = k;
        if (overflow) error = "output buffer too small";
        if (!error.empty()) {
            std::snprintf(err, errlen, "%s", error.c_str());
            return 1;
        }
        return 0;
    } catch (const std::exception &e) {
        std::snprintf(err, errlen, "%s", e.what());
        return 1;
    }
}

} // extern "C"
