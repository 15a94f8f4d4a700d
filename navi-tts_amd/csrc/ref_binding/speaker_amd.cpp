// SpeakerEncoder (model/qwen3tts/speaker.h:17-38) over the C ABI: replaces
// model/qwen3tts/speaker.hip in the reference's build.
#include "model/qwen3tts/speaker.h"

#include "amd_common.h"

namespace navi::qwen3tts {

struct SpeakerEncoder::Impl {
    navi_speaker *h = nullptr;
    navi_speaker_params sp{};
    ~Impl() { navi_speaker_destroy(h); }
};

std::unique_ptr<SpeakerEncoder> SpeakerEncoder::create(const Device &, const DeviceWeights &w, const Params &p,
                                                       double max_seconds) {
    std::unique_ptr<SpeakerEncoder> e(new SpeakerEncoder());
    e->impl_ = std::make_unique<Impl>();
    e->impl_->sp = amd::speaker_params(p);
    const std::vector<navi_tensor_ref> refs = amd::tensor_table(w);
    char err[256] = {};
    amd::check(navi_speaker_create(&e->impl_->sp, refs.data(), static_cast<int32_t>(refs.size()), max_seconds, &e->impl_->h,
                                   err, sizeof err),
               "speaker", err);
    return e;
}

SpeakerEncoder::~SpeakerEncoder() = default;

std::vector<float> SpeakerEncoder::mel(std::span<const float> wav_24k, const Params &p, int *n_frames) {
    const navi_speaker_params sp = amd::speaker_params(p);
    int32_t nf = 0;
    char err[256] = {};
    amd::check(navi_speaker_mel(&sp, wav_24k.data(), static_cast<int64_t>(wav_24k.size()), nullptr, 0, &nf, err, sizeof err),
               "speaker", err);
    std::vector<float> m(static_cast<size_t>(sp.num_mels) * static_cast<size_t>(nf));
    amd::check(navi_speaker_mel(&sp, wav_24k.data(), static_cast<int64_t>(wav_24k.size()), m.data(),
                                static_cast<int64_t>(m.size()), &nf, err, sizeof err),
               "speaker", err);
    if (n_frames) *n_frames = nf;
    return m;
}

std::vector<float> SpeakerEncoder::embed(std::span<const float> wav_24k) {
    std::vector<float> out(static_cast<size_t>(navi_speaker_dim(impl_->h)));
    char err[256] = {};
    amd::check(navi_speaker_embed(impl_->h, wav_24k.data(), static_cast<int64_t>(wav_24k.size()), out.data(), err, sizeof err),
               "speaker", err);
    return out;
}

std::vector<float> SpeakerEncoder::embed_mel(std::span<const float> mel, int n_frames) {
    if (n_frames < 0 || mel.size() < static_cast<size_t>(impl_->sp.num_mels) * static_cast<size_t>(n_frames))
        fail("speaker: mel smaller than num_mels x n_frames");
    std::vector<float> out(static_cast<size_t>(navi_speaker_dim(impl_->h)));
    char err[256] = {};
    amd::check(navi_speaker_embed_mel(impl_->h, mel.data(), n_frames, out.data(), err, sizeof err), "speaker", err);
    return out;
}

double SpeakerEncoder::last_ms() const { return navi_speaker_last_ms(impl_->h); }

} // namespace navi::qwen3tts
