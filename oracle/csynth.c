/* C restatement of oracle/synth.py's generator (same bits, OpenMP-parallel) -- test
 * infrastructure only.  Used to materialise the multi-GB synthetic checkpoints on the CPU in
 * seconds instead of minutes; tests check it against the numpy statement element for element.
 *
 *   key     = seed << 32 | stream
 *   h_w(i)  = mix64(key + (2 i + w + 1) * 0x9E3779B97F4A7C15)        w in {0, 1}
 *   S(i)    = sum of the eight 16-bit fields of h_0(i), h_1(i)
 *   value   = bf16_rne((float)(S - 262140) * scale)                  one fp32 rounding
 */
#include <stdint.h>
#include <string.h>

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline int64_t fields(uint64_t h) {
    return (int64_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48));
}

static inline uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
    return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}

/* out[j] = value(start + j), j < count */
void oracle_synth_bf16(uint16_t *out, uint64_t seed, uint64_t stream, uint64_t start,
                       uint64_t count, float scale) {
    const uint64_t key = (seed << 32) | stream;
    const uint64_t g = 0x9E3779B97F4A7C15ull;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < (int64_t)count; ++j) {
        uint64_t i = start + (uint64_t)j;
        uint64_t h0 = mix64(key + (2 * i + 1) * g);
        uint64_t h1 = mix64(key + (2 * i + 2) * g);
        int64_t s = fields(h0) + fields(h1) - 262140;
        volatile float v = (float)s * scale;   /* single IEEE multiply, no contraction */
        out[j] = bf16_rne(v);
    }
}
