// Vocoder (model/qwen3tts/vocoder.h:27-55) over the C ABI: replaces model/qwen3tts/vocoder.hip in
// the reference's build. The library makes its re-laid-out weight copies on the device from the
// arena, so DeviceWeights::upload must keep every codec tensor (vocoder_owns_tensor is false).
#include "model/qwen3tts/vocoder.h"

#include "amd_common.h"

#include <algorithm>
#include <exception>
#include <string_view>

namespace navi::qwen3tts {

bool vocoder_owns_tensor(const std::string &name) { return navi_vocoder_owns_tensor(name.c_str()) != 0; }

struct Vocoder::Impl {
    navi_vocoder *h = nullptr;
    int n_q = 16;                    // codes per frame (Params::vq_n_q)
    StageHook hook;
    std::exception_ptr hook_error;   // an exception from the hook, rethrown when decode returns
    int chunks_done = 0;             // chunks whose last stage ("pcm") the hook saw return normally
    ~Impl() { navi_vocoder_destroy(h); }
};

namespace {

// The C callback behind set_stage_hook: no exception may cross the C boundary.
void stage_trampoline(void *user, const char *name, const float *d_buf, int32_t rows, int32_t cols) {
    auto *I = static_cast<Vocoder::Impl *>(user);
    if (I->hook_error) return;
    try {
        I->hook(name, d_buf, rows, cols);
        if (std::string_view(name) == "pcm") ++I->chunks_done;
    } catch (...) {
        I->hook_error = std::current_exception();
    }
}

} // namespace

std::unique_ptr<Vocoder> Vocoder::create(const Device &, const NaviFile &, const DeviceWeights &w, const Params &p,
                                         int max_chunk_frames, int /*max_frames: decode loops over chunks without a cap*/) {
    const navi_vocoder_params vp = amd::vocoder_params(p);
    const std::vector<navi_tensor_ref> refs = amd::tensor_table(w);
    std::unique_ptr<Vocoder> v(new Vocoder());
    v->impl_ = std::make_unique<Impl>();
    v->impl_->n_q = p.vq_n_q;
    char err[256] = {};
    amd::check(navi_vocoder_create(&vp, refs.data(), static_cast<int32_t>(refs.size()), max_chunk_frames, &v->impl_->h, err,
                                   sizeof err),
               "vocoder", err);
    return v;
}

Vocoder::~Vocoder() = default;

void Vocoder::reset() { amd::check(navi_vocoder_reset(impl_->h), "vocoder reset", nullptr); }

// vocoder.hip:617-636: the codes hold n_frames x n_q values; PCM is appended chunk by chunk, so
// when the stage hook throws, out keeps only the chunks that finished before the throw.
void Vocoder::decode(std::span<const std::int32_t> codes, int n_frames, std::vector<float> &pcm) {
    if (n_frames < 0 || codes.size() < static_cast<size_t>(n_frames) * static_cast<size_t>(impl_->n_q)) {
        fail("vocoder: codes shorter than n_frames x n_q");
    }
    const size_t old = pcm.size(), spf = static_cast<size_t>(navi_vocoder_samples_per_frame(impl_->h));
    pcm.resize(old + static_cast<size_t>(n_frames) * spf);
    char err[256] = {};
    impl_->chunks_done = 0;
    const navi_status st = navi_vocoder_decode(impl_->h, codes.data(), n_frames, pcm.data() + old, err, sizeof err);
    if (impl_->hook_error) {
        std::exception_ptr e = impl_->hook_error;
        impl_->hook_error = nullptr;
        const size_t kept = std::min(static_cast<size_t>(n_frames),
                                     static_cast<size_t>(impl_->chunks_done) *
                                         static_cast<size_t>(navi_vocoder_max_chunk_frames(impl_->h)));
        pcm.resize(old + kept * spf);
        std::rethrow_exception(e);
    }
    if (st != NAVI_OK) pcm.resize(old);
    amd::check(st, "vocoder", err);
}

int Vocoder::samples_per_frame() const { return navi_vocoder_samples_per_frame(impl_->h); }
int Vocoder::max_chunk_frames() const { return navi_vocoder_max_chunk_frames(impl_->h); }
double Vocoder::last_ms() const { return navi_vocoder_last_ms(impl_->h); }

void Vocoder::set_stage_hook(StageHook hook) {
    impl_->hook = std::move(hook);
    amd::check(navi_vocoder_set_stage_hook(impl_->h, impl_->hook ? stage_trampoline : nullptr, impl_.get()),
               "vocoder stage hook", nullptr);
}

} // namespace navi::qwen3tts
