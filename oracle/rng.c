/* Plain-C restatement of the two counter generators (oracle; test infrastructure only).
 *
 * lowbias32 / counter_uniform follow engine/talker_sampler.py:60-76.
 * philox4x32_10 follows Salmon et al., SC'11 (Random123); the draw key of the
 * Philox mode (seed -> key, (step, row id) -> counter) is build-defined.
 * Built by oracle/Makefile into oracle/_build/liboracle_rng.so and loaded by
 * the tests with ctypes.
 */
#include <stdint.h>

static uint32_t lowbias32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

uint32_t oracle_lowbias32(uint32_t x) { return lowbias32(x); }

uint32_t oracle_counter_hash(int64_t seed, int64_t step) {
    uint64_t s = (uint64_t)seed, t = (uint64_t)step;
    uint32_t h = lowbias32((uint32_t)s);
    h = lowbias32(h ^ (uint32_t)(s >> 32) ^ 0x9E3779B9u);
    return lowbias32(h ^ (uint32_t)t ^ 0x632BE5ABu);
}

static float to_unit(uint32_t w) { return (float)(w >> 8) * (1.0f / 16777216.0f); }

float oracle_counter_uniform(int64_t seed, int64_t step) { return to_unit(oracle_counter_hash(seed, step)); }

void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float oracle_philox_uniform(int64_t seed, int64_t step, int64_t row_id) {
    uint64_t s = (uint64_t)seed, t = (uint64_t)step, r = (uint64_t)row_id;
    uint32_t ctr[4] = {(uint32_t)t, (uint32_t)(t >> 32), (uint32_t)r, (uint32_t)(r >> 32)};
    uint32_t key[2] = {(uint32_t)s, (uint32_t)(s >> 32)};
    uint32_t out[4];
    oracle_philox4x32_10(ctr, key, out);
    return to_unit(out[0]);
}
