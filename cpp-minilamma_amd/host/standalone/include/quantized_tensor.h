// quantized_tensor.h -- stand-in for the part of the reference's
// quantized-tensor header this library uses (GGUF-style 32-element block
// formats), found only when the library is built on its own: inside the
// reference tree its own include/quantized_tensor.h is found instead.
//
// Same enumerators, constants and packed block layouts as the reference
// (include/quantized_tensor.h:10-36 of the reference tree): the quantized
// gather reads these bytes as they are.  All multi-byte fields are
// little-endian IEEE binary16; in Q4 blocks byte i holds element i in its
// low nibble and element i + 16 in its high nibble.
#pragma once
#include <cstddef>
#include <cstdint>

namespace yan_lamma {
constexpr size_t kQuantBlockSize = 32;
constexpr size_t kBytesPerQ80Block = 34;  // fp16 scale + 32 int8
constexpr size_t kBytesPerQ40Block = 18;  // fp16 scale + 16 nibble bytes
constexpr size_t kBytesPerQ41Block = 20;  // fp16 scale + fp16 min + 16 nibble bytes
enum class QuantType {
    kF32,
    kF16,
    kQ80,
    kQ40,
    kQ41,
};
struct Block_Q80 {
    uint16_t d;
    int8_t qs[32];
};
struct Block_Q40 {
    uint16_t d;
    uint8_t qs[16];
};
struct Block_Q41 {
    uint16_t d;
    uint16_t m;
    uint8_t qs[16];
};
static_assert(sizeof(Block_Q80) == kBytesPerQ80Block, "Q8_0 block must be 34 bytes");
static_assert(sizeof(Block_Q40) == kBytesPerQ40Block, "Q4_0 block must be 18 bytes");
static_assert(sizeof(Block_Q41) == kBytesPerQ41Block, "Q4_1 block must be 20 bytes");
}  // namespace yan_lamma
