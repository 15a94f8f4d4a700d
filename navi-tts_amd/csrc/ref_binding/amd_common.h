// Shared conversions for the reference-side forwarders (frame_amd.cpp, talker_amd.cpp,
// vocoder_amd.cpp, speaker_amd.cpp): the reference's Params and DeviceWeights as the C ABI's
// navi_model_params / navi_vocoder_params / navi_speaker_params and navi_tensor_ref table.
//
// These files are compiled INTO the reference's build in place of model/qwen3tts/{frame,talker,
// vocoder,speaker}.hip (they include its headers: model/qwen3tts/*.h, runtime/...), and link
// against libnavi_amd.so. They are not part of this repository's own build.
#pragma once

#include "model/qwen3tts/params.h"
#include "navi_amd.h"
#include "runtime/common/error.h"
#include "runtime/weights/device_weights.h"

#include <string>
#include <vector>

namespace navi::qwen3tts::amd {

inline navi_xformer_params xformer(const TransformerParams &t) {
    return {t.hidden, t.n_layer, t.n_head, t.n_kv_head, t.head_dim, t.ff, t.vocab, t.rms_eps, t.rope_theta};
}

// params.h:29-73 -> the fields the frame and the talker read (params.cpp:59-96).
inline navi_model_params model_params(const Params &p) {
    navi_model_params m{};
    m.talker = xformer(p.talker);
    m.cp = xformer(p.cp);
    m.n_code_groups = p.n_code_groups;
    m.codec_eos_id = p.codec_eos_id;
    m.text_hidden = p.text_hidden;
    m.text_vocab = p.text_vocab;
    m.tts_bos_id = p.tts_bos_id;
    m.tts_eos_id = p.tts_eos_id;
    m.tts_pad_id = p.tts_pad_id;
    m.codec_bos_id = p.codec_bos_id;
    m.codec_pad_id = p.codec_pad_id;
    m.codec_think_id = p.codec_think_id;
    m.codec_nothink_id = p.codec_nothink_id;
    m.codec_think_bos_id = p.codec_think_bos_id;
    m.codec_think_eos_id = p.codec_think_eos_id;
    return m;
}

// params.cpp:106-117: the codec decoder.
inline navi_vocoder_params vocoder_params(const Params &p) {
    if (p.vocoder_upsampling_ratios.size() != 2 || p.vocoder_upsample_rates.size() != 4)
        fail("vocoder: expected 2 upsampling ratios and 4 upsample rates");
    navi_vocoder_params v{};
    v.xf = xformer(p.vocoder);
    v.latent_dim = p.vq_latent;
    v.codebook_dim = p.vq_codebook_dim;
    v.codebook_size = p.vq_codebook_size;
    v.n_q = p.vq_n_q;
    v.n_semantic = p.vq_n_semantic;
    v.decoder_dim = p.vocoder_decoder_dim;
    v.sliding_window = p.vocoder_sliding_window;
    for (int i = 0; i < 2; ++i) v.upsampling_ratios[i] = p.vocoder_upsampling_ratios[i];
    for (int i = 0; i < 4; ++i) v.upsample_rates[i] = p.vocoder_upsample_rates[i];
    v.samples_per_frame = p.codec_upsample;
    return v;
}

// params.cpp:97-104: the speaker encoder and its mel front end.
inline navi_speaker_params speaker_params(const Params &p) {
    return {p.spk_sample_rate, p.spk_dim, p.mel_n_fft, p.mel_num_mels, p.mel_hop, p.mel_win, p.mel_fmin, p.mel_fmax};
}

inline int32_t dtype_code(DType d) {
    switch (d) {
    case DType::F32: return NAVI_DT_F32;
    case DType::F16: return NAVI_DT_F16;
    case DType::BF16: return NAVI_DT_BF16;
    case DType::I32: return NAVI_DT_I32;
    case DType::U8: return NAVI_DT_U8;
    }
    return -1;
}

// Every tensor of the arena by name (DeviceWeights::tensors, device_weights.h:53): the C ABI binds
// what it needs from this table. The names point into w's map, so the table lives as long as w.
inline std::vector<navi_tensor_ref> tensor_table(const DeviceWeights &w) {
    std::vector<navi_tensor_ref> refs;
    refs.reserve(w.tensors().size());
    for (const auto &[name, t] : w.tensors()) {
        navi_tensor_ref r{};
        r.name = name.c_str();
        r.ptr = t.ptr;
        r.dtype = dtype_code(t.info.dtype);
        r.ndim = static_cast<int32_t>(t.info.dims.size());
        if (r.ndim > 4) fail("weights: tensor '" + name + "' has more than 4 dimensions");
        for (int i = 0; i < r.ndim; ++i) r.dims[i] = t.info.dims[static_cast<size_t>(i)];
        refs.push_back(r);
    }
    return refs;
}

// Setup calls throw navi::Error (error.h:10-14) with the library's message.
inline void check(navi_status st, const char *who, const char *err) {
    if (st != NAVI_OK) fail(std::string(who) + ": " + (err && *err ? err : "failed"));
}

} // namespace navi::qwen3tts::amd
