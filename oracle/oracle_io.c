/* cpuforge on-disk-format oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatements of the reference's 16-bit float conversions, the
 * checker of cfio_bf16_to_f32 / cfio_f16_to_f32 and of the widening inside
 * cfio_st_read_f32 (include/cfio.h).  Nothing in the product links or calls
 * this file.  Pinned in tests/test_oracle_io.py against the reference's own
 * known-answer tests (crates/io/src/dtype.rs:36-57) and, over all 65536
 * patterns, against numpy's half-precision conversion.
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

static float from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

/* crates/io/src/dtype.rs:3-5 */
void orc_bf16_to_f32(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = from_bits((uint32_t)src[i] << 16);
}

/* crates/io/src/dtype.rs:7-33, with the reference's shift loop for subnormals. */
void orc_f16_to_f32(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const uint16_t h = src[i];
        const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
        uint32_t bits;
        if (exp == 0) {
            if (man == 0) {
                bits = sign << 31;
            } else {
                uint32_t e = 113, m = man;
                while ((m & 0x400u) == 0) {
                    m <<= 1;
                    e -= 1;
                }
                bits = (sign << 31) | (e << 23) | ((m & 0x3ffu) << 13);
            }
        } else if (exp == 0x1f) {
            bits = (sign << 31) | (0xffu << 23) | (man << 13);
        } else {
            bits = (sign << 31) | ((exp + 127 - 15) << 23) | (man << 13);
        }
        dst[i] = from_bits(bits);
    }
}
