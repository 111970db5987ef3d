// Weight-name conventions: scoring and rewrite rules of WeightNameMapper.swift.
#include "weight_names.hpp"

#include <algorithm>

namespace mnn {
namespace {

bool starts(const std::string& s, const char* p) { return s.rfind(p, 0) == 0; }
bool has(const std::string& s, const char* p) { return s.find(p) != std::string::npos; }

// Every non-overlapping occurrence, scanned left to right (Foundation's replacingOccurrences).
std::string replace_all(std::string s, const std::string& from, const std::string& to) {
  std::string out;
  size_t at = 0;
  for (size_t hit; (hit = s.find(from, at)) != std::string::npos; at = hit + from.size())
    out.append(s, at, hit - at).append(to);
  return out.append(s, at, std::string::npos);
}

// remapTransformerSublayer (:258-295): the sub-layer's time/freq-specific name.
std::string remap_sublayer(const std::string& sub, const std::string& path) {
  if (starts(sub, "linear1.") || starts(sub, "linear2.")) return "ffn_" + path + "." + sub;
  static const char* const renamed[] = {"self_attn", "cross_attn", "norm1", "norm2", "norm3"};
  for (const char* stem : renamed) {
    const std::string prefix = std::string(stem) + ".";
    if (starts(sub, prefix.c_str())) return stem + ("_" + path) + "." + sub.substr(prefix.size());
  }
  return sub + "_" + path;
}

// True when "cross_transformer.layers_t.<digits>." occurs anywhere in s.
bool has_time_layer(const std::string& s) {
  static const std::string key = "cross_transformer.layers_t.";
  for (size_t at = s.find(key); at != std::string::npos; at = s.find(key, at + 1)) {
    size_t i = at + key.size(), d = i;
    while (d < s.size() && s[d] >= '0' && s[d] <= '9') ++d;
    if (d > i && d < s.size() && s[d] == '.') return true;
  }
  return false;
}

// remapCrossTransformerName (:225-255). As in the reference the level is read from just after
// the fixed prefix at the start of the name once the pattern is found.
std::string remap_cross(const std::string& name) {
  static const std::string tprefix = "cross_transformer.layers_t.";
  static const std::string fprefix = "cross_transformer.layers.";
  const std::string* prefix = nullptr;
  const char* path = nullptr;
  if (has_time_layer(name)) {
    prefix = &tprefix;
    path = "time";
  } else if (starts(name, fprefix.c_str()) && !has(name, ".layers_t.")) {
    prefix = &fprefix;
    path = "freq";
  }
  if (!prefix || name.size() < prefix->size()) return name;
  const std::string after = name.substr(prefix->size());
  const size_t dot = after.find('.');
  if (dot == std::string::npos) return name;
  return fprefix + after.substr(0, dot) + "." + remap_sublayer(after.substr(dot + 1), path);
}

}  // namespace

WeightConvention detect_convention(const std::vector<std::string>& names) {
  int demucs = 0, metal = 0;
  for (const std::string& n : names) {
    if (starts(n, "tencoder.") || starts(n, "tdecoder.")) demucs += 2;
    if (starts(n, "crosstransformer.")) demucs += 2;
    if (has(n, ".conv_tr.")) demucs += 1;
    if (has(n, ".norm1.") || has(n, ".norm2.")) demucs += 1;
    if (starts(n, "channel_upsampler.") || starts(n, "channel_downsampler.")) demucs += 1;
    if (starts(n, "time_encoder.") || starts(n, "time_decoder.")) metal += 2;
    if (starts(n, "freq_encoder.") || starts(n, "freq_decoder.")) metal += 2;
    if (starts(n, "cross_transformer.")) metal += 2;
    if (has(n, ".conv_transpose.")) metal += 1;
    if (has(n, "_to_transformer.") || has(n, "transformer_to_")) metal += 1;
    if (has(n, ".self_attn_freq.") || has(n, ".self_attn_time.")) metal += 1;
  }
  if (metal > demucs && metal >= 3) return WC_METALAUDIO;
  if (demucs > metal && demucs >= 3) return WC_DEMUCS;
  return WC_UNKNOWN;
}

std::string demucs_to_metalaudio(const std::string& name) {
  std::string r = name;
  if (starts(r, "tencoder.")) {
    r = replace_all(replace_all(r, "tencoder.", "time_encoder."), ".norm1.", ".norm.");
  } else if (starts(r, "tdecoder.")) {
    r = replace_all(r, "tdecoder.", "time_decoder.");
    r = replace_all(replace_all(r, ".conv_tr.", ".conv_transpose."), ".norm2.", ".norm.");
  } else if (starts(r, "encoder.")) {
    r = replace_all(replace_all(r, "encoder.", "freq_encoder."), ".norm1.", ".norm.");
  } else if (starts(r, "decoder.")) {
    r = replace_all(r, "decoder.", "freq_decoder.");
    r = replace_all(replace_all(r, ".conv_tr.", ".conv_transpose."), ".norm2.", ".norm.");
  } else if (starts(r, "channel_upsampler.")) {
    r = replace_all(r, "channel_upsampler.", "freq_to_transformer.");
  } else if (starts(r, "channel_downsampler.")) {
    r = replace_all(r, "channel_downsampler.", "transformer_to_freq.");
  } else if (starts(r, "channel_upsampler_t.")) {
    r = replace_all(r, "channel_upsampler_t.", "time_to_transformer.");
  } else if (starts(r, "channel_downsampler_t.")) {
    r = replace_all(r, "channel_downsampler_t.", "transformer_to_time.");
  } else if (starts(r, "crosstransformer.")) {
    r = remap_cross(replace_all(r, "crosstransformer.", "cross_transformer."));
  }
  return r;
}

std::string metalaudio_to_demucs(const std::string& name) {
  std::string r = name;
  if (starts(r, "time_encoder.")) {
    r = replace_all(replace_all(r, "time_encoder.", "tencoder."), ".norm.", ".norm1.");
  } else if (starts(r, "time_decoder.")) {
    r = replace_all(r, "time_decoder.", "tdecoder.");
    r = replace_all(replace_all(r, ".conv_transpose.", ".conv_tr."), ".norm.", ".norm2.");
  } else if (starts(r, "freq_encoder.")) {
    r = replace_all(replace_all(r, "freq_encoder.", "encoder."), ".norm.", ".norm1.");
  } else if (starts(r, "freq_decoder.")) {
    r = replace_all(r, "freq_decoder.", "decoder.");
    r = replace_all(replace_all(r, ".conv_transpose.", ".conv_tr."), ".norm.", ".norm2.");
  } else if (starts(r, "freq_to_transformer.")) {
    r = replace_all(r, "freq_to_transformer.", "channel_upsampler.");
  } else if (starts(r, "transformer_to_freq.")) {
    r = replace_all(r, "transformer_to_freq.", "channel_downsampler.");
  } else if (starts(r, "time_to_transformer.")) {
    r = replace_all(r, "time_to_transformer.", "channel_upsampler_t.");
  } else if (starts(r, "transformer_to_time.")) {
    r = replace_all(r, "transformer_to_time.", "channel_downsampler_t.");
  } else if (starts(r, "cross_transformer.")) {
    r = replace_all(r, "cross_transformer.", "crosstransformer.");
  }
  return r;
}

std::string to_metalaudio(WeightConvention from, const std::string& name) {
  return from == WC_DEMUCS ? demucs_to_metalaudio(name) : name;
}

std::string from_metalaudio(const std::string& name, WeightConvention to) {
  return to == WC_DEMUCS ? metalaudio_to_demucs(name) : name;
}

bool is_metalaudio_naming(const std::string& n) {
  for (const char* p : {"time_encoder.", "time_decoder.", "freq_encoder.", "freq_decoder.",
                        "cross_transformer.", "time_to_transformer.", "freq_to_transformer."})
    if (starts(n, p)) return true;
  return false;
}

bool is_demucs_naming(const std::string& n) {
  for (const char* p : {"tencoder.", "tdecoder.", "crosstransformer.", "channel_upsampler."})
    if (starts(n, p)) return true;
  return false;
}

std::string find_mapped(const std::vector<std::string>& available, WeightConvention conv,
                        const std::string& metalaudio_name) {
  const auto present = [&](const std::string& n) {
    return std::binary_search(available.begin(), available.end(), n);
  };
  if (conv == WC_METALAUDIO) return present(metalaudio_name) ? metalaudio_name : std::string();
  const std::string original = from_metalaudio(metalaudio_name, conv);
  if (present(original)) return original;
  for (const std::string& n : available)
    if (to_metalaudio(conv, n) == metalaudio_name) return n;
  return std::string();
}

}  // namespace mnn
