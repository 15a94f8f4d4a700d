// Test harness (not the product): reads a .navi with the reference's own reader and parameter
// table, and prints what they see, one record per line, for tests/test_ref_reader.py.
//
// Built by that test from this file plus the reference's runtime/weights/navi_file.cpp and
// model/qwen3tts/params.cpp, compiled where they lie under /root/reference (never copied).
// Calls: NaviFile::open (navi_file.cpp:79-148), read_params (params.cpp:59-130) and
// validate (params.cpp:286-303).
//
// Output lines:
//   P <key> <value...>                 a field of the Params read_params returned
//   MISSING <name> | MISMATCH <text> | UNUSED <name>
//   T <name> <dtype> <ndim> <dims...> <offset> <nbytes> <sum> <wsum>
//     sum  = sum of the tensor's bytes as little-endian u64 words (zero-padded), mod 2^64
//     wsum = sum of word[i] * (2i + 1), mod 2^64
//   OK | ERROR <message>

#include "model/qwen3tts/params.h"
#include "runtime/common/error.h"
#include "runtime/weights/navi_file.h"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

using navi::NaviFile;
using navi::qwen3tts::Params;
using navi::qwen3tts::TransformerParams;

namespace {

void xf(const char * ns, const TransformerParams & t) {
    std::printf("P %s.hidden %d\nP %s.n_layer %d\nP %s.n_head %d\nP %s.n_kv_head %d\nP %s.head_dim %d\n"
                "P %s.ff %d\nP %s.rms_eps %.9g\nP %s.rope_theta %.17g\nP %s.vocab %d\nP %s.max_pos %d\n",
                ns, t.hidden, ns, t.n_layer, ns, t.n_head, ns, t.n_kv_head, ns, t.head_dim, ns, t.ff, ns,
                static_cast<double>(t.rms_eps), ns, t.rope_theta, ns, t.vocab, ns, t.max_pos);
}

void ints(const char * key, const std::vector<int> & v) {
    std::printf("P %s", key);
    for (int x : v) std::printf(" %d", x);
    std::printf("\n");
}

void print_params(const Params & p) {
    std::printf("P name %s\nP dtype %s\n", p.name.c_str(), p.dtype.c_str());
    std::printf("P im_start_id %d\nP im_end_id %d\nP assistant_id %d\nP tts_bos_id %d\nP tts_eos_id %d\n"
                "P tts_pad_id %d\nP text_vocab %d\nP text_hidden %d\n",
                p.im_start_id, p.im_end_id, p.assistant_id, p.tts_bos_id, p.tts_eos_id, p.tts_pad_id,
                p.text_vocab, p.text_hidden);
    xf("talker", p.talker);
    std::printf("P n_code_groups %d\nP position_id_per_second %d\nP mrope_interleaved %d\n", p.n_code_groups,
                p.position_id_per_second, p.mrope_interleaved ? 1 : 0);
    ints("mrope_section", p.mrope_section);
    std::printf("P codec_bos_id %d\nP codec_eos_id %d\nP codec_pad_id %d\nP codec_think_id %d\n"
                "P codec_nothink_id %d\nP codec_think_bos_id %d\nP codec_think_eos_id %d\n",
                p.codec_bos_id, p.codec_eos_id, p.codec_pad_id, p.codec_think_id, p.codec_nothink_id,
                p.codec_think_bos_id, p.codec_think_eos_id);
    for (const auto & [lang, id] : p.language_ids) std::printf("P language.%s %d\n", lang.c_str(), id);
    xf("cp", p.cp);
    std::printf("P spk_dim %d\nP spk_sample_rate %d\nP mel_n_fft %d\nP mel_num_mels %d\nP mel_hop %d\n"
                "P mel_win %d\nP mel_fmin %.9g\nP mel_fmax %.9g\n",
                p.spk_dim, p.spk_sample_rate, p.mel_n_fft, p.mel_num_mels, p.mel_hop, p.mel_win,
                static_cast<double>(p.mel_fmin), static_cast<double>(p.mel_fmax));
    std::printf("P codec_sample_rate %d\nP codec_upsample %d\n", p.codec_sample_rate, p.codec_upsample);
    xf("vocoder", p.vocoder);
    std::printf("P vq_latent %d\nP vq_codebook_dim %d\nP vq_codebook_size %d\nP vq_n_q %d\nP vq_n_semantic %d\n"
                "P vocoder_decoder_dim %d\nP vocoder_sliding_window %d\nP has_codec_encoder %d\n",
                p.vq_latent, p.vq_codebook_dim, p.vq_codebook_size, p.vq_n_q, p.vq_n_semantic,
                p.vocoder_decoder_dim, p.vocoder_sliding_window, p.has_codec_encoder ? 1 : 0);
    ints("vocoder_upsample_rates", p.vocoder_upsample_rates);
    ints("vocoder_upsampling_ratios", p.vocoder_upsampling_ratios);
    std::printf("P temperature %.9g\nP top_p %.9g\nP repetition_penalty %.9g\nP top_k %d\n"
                "P cp_temperature %.9g\nP cp_top_p %.9g\nP cp_top_k %d\n",
                static_cast<double>(p.temperature), static_cast<double>(p.top_p),
                static_cast<double>(p.repetition_penalty), p.top_k, static_cast<double>(p.cp_temperature),
                static_cast<double>(p.cp_top_p), p.cp_top_k);
}

void print_tensor(const NaviFile & f, const navi::TensorInfo & t) {
    const auto * b = static_cast<const unsigned char *>(f.data(t));
    std::uint64_t sum = 0, wsum = 0;
    const std::uint64_t n_words = (t.nbytes + 7) / 8;
    for (std::uint64_t i = 0; i < n_words; ++i) {
        std::uint64_t w = 0;
        const std::uint64_t at = i * 8;
        std::memcpy(&w, b + at, t.nbytes - at >= 8 ? 8 : static_cast<std::size_t>(t.nbytes - at));
        sum += w;
        wsum += w * (2 * i + 1);
    }
    std::printf("T %s %s %zu", t.name.c_str(), navi::dtype_name(t.dtype), t.dims.size());
    for (auto d : t.dims) std::printf(" %llu", static_cast<unsigned long long>(d));
    std::printf(" %llu %llu %llu %llu\n", static_cast<unsigned long long>(t.offset),
                static_cast<unsigned long long>(t.nbytes), static_cast<unsigned long long>(sum),
                static_cast<unsigned long long>(wsum));
}

} // namespace

int main(int argc, char ** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s file.navi\n", argv[0]);
        return 2;
    }
    try {
        const NaviFile f = NaviFile::open(argv[1]);
        const Params p = navi::qwen3tts::read_params(f);
        print_params(p);
        const auto v = navi::qwen3tts::validate(f, p);
        for (const auto & s : v.missing) std::printf("MISSING %s\n", s.c_str());
        for (const auto & s : v.shape_mismatch) std::printf("MISMATCH %s\n", s.c_str());
        for (const auto & s : v.unused) std::printf("UNUSED %s\n", s.c_str());
        for (const auto & t : f.tensors()) print_tensor(f, t);
        std::printf("OK\n");
    } catch (const std::exception & e) {
        std::printf("ERROR %s\n", e.what());
        return 1;
    }
    return 0;
}
