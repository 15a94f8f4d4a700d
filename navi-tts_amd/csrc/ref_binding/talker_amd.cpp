// Talker (model/qwen3tts/talker.h:34-67) over the C ABI: replaces model/qwen3tts/talker.hip in
// the reference's build. The KV cache is the library's (f16 [max_positions][kv_dim] per layer,
// talker.h:20-24); kv() exposes it in the reference's KvCache form for Frame::run.
#include "model/qwen3tts/talker.h"

#include "amd_common.h"

namespace navi::qwen3tts {

struct Talker::Impl {
    navi_talker *h = nullptr;
    Params p;
    KvCache kv;
    Prompt prompt;
    ~Impl() { navi_talker_destroy(h); }
};

std::unique_ptr<Talker> Talker::create(const Device &, const DeviceWeights &w, const Params &p, int max_prompt_tokens,
                                       int max_positions) {
    const navi_model_params mp = amd::model_params(p);
    const std::vector<navi_tensor_ref> refs = amd::tensor_table(w);
    std::unique_ptr<Talker> t(new Talker());
    t->impl_ = std::make_unique<Impl>();
    Impl &I = *t->impl_;
    I.p = p;
    char err[256] = {};
    amd::check(navi_talker_create(&mp, refs.data(), static_cast<int32_t>(refs.size()), max_prompt_tokens, max_positions,
                                  &I.h, err, sizeof err),
               "talker", err);
    navi_kv_view view{};
    int32_t n_used = 0;
    amd::check(navi_talker_kv(I.h, &view, &n_used), "talker kv", nullptr);
    I.kv.n_layer = view.n_layer;
    I.kv.max_pos = view.max_pos;
    I.kv.kv_dim = view.kv_dim;
    I.kv.k.assign(view.k, view.k + view.n_layer);
    I.kv.v.assign(view.v, view.v + view.n_layer);
    I.kv.n_used = n_used;
    return t;
}

Talker::~Talker() = default;

// The library's projections take q, k, v (and gate, up) as separate weights: no arena adjacency
// is needed, so no groups are requested.
DeviceWeights::Groups Talker::fused_groups(const Params &) { return {}; }

const Prompt &Talker::build_prompt(std::span<const std::int32_t> ids, const std::string &language,
                                   std::span<const float> speaker) {
    Impl &I = *impl_;
    if (static_cast<int>(speaker.size()) != I.p.talker.hidden) fail("talker: speaker embedding must be [hidden]");
    int32_t lang = -1;                                  // "" / "auto": no language row (talker.hip:304-312)
    if (!language.empty() && language != "auto") {
        const auto it = I.p.language_ids.find(language);
        if (it == I.p.language_ids.end()) fail("talker: unknown language '" + language + "'");
        lang = it->second;
    }
    navi_prompt np{};
    char err[256] = {};
    amd::check(navi_talker_build_prompt(I.h, ids.data(), static_cast<int32_t>(ids.size()), lang, speaker.data(), &np, err,
                                        sizeof err),
               "talker", err);
    I.prompt.prefill = const_cast<float *>(np.prefill);
    I.prompt.trailing = const_cast<float *>(np.trailing);
    I.prompt.tts_pad = const_cast<float *>(np.tts_pad);
    I.prompt.n_prefill = np.n_prefill;
    I.prompt.n_trailing = np.n_trailing;
    return I.prompt;
}

void Talker::prefill(const Prompt &prompt) {
    Impl &I = *impl_;
    char err[256] = {};
    amd::check(navi_talker_prefill(I.h, prompt.prefill, prompt.n_prefill, err, sizeof err), "talker", err);
    I.kv.n_used = prompt.n_prefill;                     // talker.hip:398
}

KvCache &Talker::kv() { return impl_->kv; }
const float *Talker::d_hidden() const { return navi_talker_hidden(impl_->h); }
const float *Talker::d_logits() const { return navi_talker_logits(impl_->h); }
double Talker::last_ms() const { return navi_talker_last_ms(impl_->h); }

} // namespace navi::qwen3tts
