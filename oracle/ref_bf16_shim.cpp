// C entry points over the reference's alveare::bf16 (runtime/cpp/src/bf16.cpp),
// so that the oracle's bf16 conversion can be checked against the reference's
// own compiled code. Test infrastructure only.
#include <cstdint>

#include "alveare/bf16.h"

extern "C" uint16_t ref_bf16_from_f32(float f) { return alveare::bf16(f).v; }

extern "C" float ref_f32_from_bf16(uint16_t h) {
    alveare::bf16 b;
    b.v = h;
    return b.to_float();
}
