// Weight-name conventions (WeightNameMapper.swift:7-422): detection of the MetalAudio or Demucs
// naming from a file's tensor names, and the name rewrites between them. Host-only string work.
// Matching is on bytes; the reference matches canonically equivalent Unicode sequences, which is
// the same thing for the ASCII names both conventions use.
#pragma once

#include <string>
#include <vector>

namespace mnn {

enum WeightConvention { WC_METALAUDIO = 0, WC_DEMUCS = 1, WC_UNKNOWN = 2 };

// detectConvention(from:) (WeightNameMapper.swift:83-137): pattern scores, winner needs >= 3.
WeightConvention detect_convention(const std::vector<std::string>& names);
// demucsToMetalAudio (:177-222) and metalAudioToDemucs (:300-342).
std::string demucs_to_metalaudio(const std::string& name);
std::string metalaudio_to_demucs(const std::string& name);
// toMetalAudio(name:) (:148-157) / fromMetalAudio(name:to:) (:165-174).
std::string to_metalaudio(WeightConvention from, const std::string& name);
std::string from_metalaudio(const std::string& name, WeightConvention to);
bool is_metalaudio_naming(const std::string& name);  // :372-380
bool is_demucs_naming(const std::string& name);      // :383-388
// loadTensorMapped's lookup (:404-420): the name in `available` (sorted) that holds the tensor
// `metalaudio_name` names; empty when none does.
std::string find_mapped(const std::vector<std::string>& available, WeightConvention conv,
                        const std::string& metalaudio_name);

}  // namespace mnn
