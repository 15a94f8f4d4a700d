// Frame (model/qwen3tts/frame.h:46-71) over the C ABI: replaces model/qwen3tts/frame.hip in the
// reference's build. Per-frame failures are returned in FrameResult, never thrown (frame.hip:
// 653-681, 787-810); setup failures throw navi::Error.
#include "model/qwen3tts/frame.h"

#include "amd_common.h"

#include <algorithm>

namespace navi::qwen3tts {

struct Frame::Impl {
    navi_frame *h = nullptr;
    ~Impl() { navi_frame_destroy(h); }
};

namespace {

navi_sampling sampling(const Sampling &s) {
    return {s.temperature, s.top_k, s.repetition_penalty, s.cp_temperature, s.cp_top_k, s.min_frames};
}

FrameResult result(const navi_frame_result &r) {
    FrameResult out;
    out.ok = r.ok != 0;
    out.eos = r.eos != 0;
    std::copy(r.codes, r.codes + 16, out.codes);
    out.us = r.us;
    if (!out.ok) out.error = r.error;
    return out;
}

} // namespace

std::unique_ptr<Frame> Frame::create(const Device &, const DeviceWeights &w, const Params &p, const FrameOptions &opt) {
    const navi_model_params mp = amd::model_params(p);
    const std::vector<navi_tensor_ref> refs = amd::tensor_table(w);
    // The reference's spin cap counts barrier spins (~10 ns each, 50M ~ 0.5 s); a wait here polls a
    // coherent word (~0.25-0.5 us per poll), so the same time budget is about 1/25 of the count.
    const navi_frame_options fo{opt.blocks_per_mp, std::max<unsigned long long>(1ull, opt.spin_cap / 25ull)};
    std::unique_ptr<Frame> f(new Frame());
    f->impl_ = std::make_unique<Impl>();
    char err[256] = {};
    amd::check(navi_frame_create(&mp, refs.data(), static_cast<int32_t>(refs.size()), &fo, &f->impl_->h, err, sizeof err),
               "frame", err);
    return f;
}

Frame::~Frame() = default;

void Frame::reset() { amd::check(navi_frame_reset(impl_->h), "frame reset", nullptr); }

FrameResult Frame::run_first(const float *d_hidden, const float *d_logits, const float *d_trailing, const Sampling &s,
                             std::uint64_t seed, int frame_index) {
    const navi_sampling ns = sampling(s);
    navi_frame_result r{};
    navi_frame_run(impl_->h, nullptr, 0, 1, d_hidden, d_logits, d_trailing, &ns, seed, frame_index, &r);
    return result(r);
}

FrameResult Frame::run(KvCache &kv, int n_past, const float *d_trailing, const Sampling &s, std::uint64_t seed,
                       int frame_index) {
    const navi_kv_view view{kv.n_layer, kv.max_pos, kv.kv_dim, kv.k.data(), kv.v.data()};
    const navi_sampling ns = sampling(s);
    navi_frame_result r{};
    navi_frame_run(impl_->h, &view, n_past, 0, nullptr, nullptr, d_trailing, &ns, seed, frame_index, &r);
    if (r.ok) kv.n_used = n_past + 1;                    // frame.hip:808
    return result(r);
}

const float *Frame::d_step_out() const { return navi_frame_step_out(impl_->h); }
int Frame::grid_blocks() const { return navi_frame_grid_blocks(impl_->h); }
int Frame::occupancy_per_mp() const { return navi_frame_occupancy_per_mp(impl_->h); }

} // namespace navi::qwen3tts
