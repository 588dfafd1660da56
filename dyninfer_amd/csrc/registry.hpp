// Kernel-registry restatement (see registry.cpp).
#pragma once
#include <string>

namespace dmx {

// JSON array of this library's gfx950 KernelCandidateDescriptors.
const std::string& candidates_json();

// Returns 0 on success (out = SelectionReport, or SelectedKernelCandidate when
// `require`), 1 on malformed input / duplicate ids, 2 when `require` finds no
// candidate (err = the E_KERNEL_COVERAGE message).
int registry_select(const char* candidates, const char* request_json, const char* target_json, bool require,
                    std::string& out, std::string& err);

// The compiler's precision gate over a SelectedKernelCandidate, relaxed for
// bf16 activations: 0 = accepted, 1 = malformed input, 2 = rejected (err =
// the lower.precision message).
int precision_check(const char* selected_json, const char* activation_type, std::string& err);

}  // namespace dmx
