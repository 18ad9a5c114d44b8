// Prints the reference's bf16 -> u8 pack (render/kernels/dataflow/img_pack_u8.h,
// compiled from the reference's own header) for all 65536 bf16 bit patterns,
// one per line. TEST INFRASTRUCTURE ONLY: tests/test_oracle_kats.py compares
// it with oracle.pack_u8.
#include <cstdint>
#include <cstdio>

#include "img_pack_u8.h"

int main() {
    for (uint32_t b = 0; b < 65536u; ++b) std::printf("%u\n", img_pack_u8::bf16_to_u8(b));
    return 0;
}
