// C-ABI shim over the reference's own host dequant and fp16 codecs, so the
// oracle can be checked against them.  TEST INFRASTRUCTURE ONLY: built into
// oracle/_ref/ from the reference sources where they lie (see Makefile); it is
// never linked by the product library.
//   GGUFLoader::dequant_block_f32 -> src/gguf.cpp:566-571 (decl gguf.hpp:87)
//   fp16_to_float / float_to_fp16 -> include/nanovllm/common.hpp:28-91
#include <cstdint>
#include <string>

#include "nanovllm/common.hpp"
#include "nanovllm/gguf.hpp"

extern "C" int ref_dequant_block_f32(const char* dtype, const uint8_t* blk, float* y) {
  return GGUFLoader::dequant_block_f32(std::string(dtype), blk, y) ? 1 : 0;
}
extern "C" float ref_fp16_to_float(uint16_t h) { return fp16_to_float(h); }
extern "C" uint16_t ref_float_to_fp16(float f) { return float_to_fp16(f); }
