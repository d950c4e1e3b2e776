// Binding shim for the reference's own host primitives — TEST INFRASTRUCTURE ONLY.
//
// Compiled together with the reference source file src/qwen3_primitives.cpp,
// straight from /root/reference (never copied), into oracle/_ref/.  It only
// re-exports two reference functions with C linkage so the tests can check the
// oracle's restatement against the real code:
//   fp16_bits_to_float  (src/qwen3_primitives.cpp:67-91)
//   softmax_reference   (src/qwen3_primitives.cpp:137-146)
#include "miinfer/qwen3_primitives.hpp"

#include <cstddef>
#include <cstdint>

extern "C" float miikv_ref_fp16_bits_to_float(std::uint16_t bits) {
    return miinfer::fp16_bits_to_float(bits);
}

extern "C" void miikv_ref_softmax(const float* input, float* output, std::size_t n) {
    miinfer::softmax_reference({input, n}, {output, n});
}
