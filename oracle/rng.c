/* ORACLE — test infrastructure only. Nothing in the product path may link, load or call this file.
 *
 * CPU restatement of noise_amd's counter-based perturbation noise, the replacement this build defines for the
 * reference's torch.randn noise buffer and torch.randint offsets:
 *   - archive/10M/train/val/eggroll.py:35   NOISE = 2**28 values in one fixed Gaussian buffer
 *   - archive/10M/train/val/eggroll.py:114  buffer = torch.randn(NOISE, generator=manual_seed(SEED))
 *   - archive/10M/train/val/eggroll.py:117-120  offsets: generator seeded 1_000_003*SEED + step, one
 *                                        randint(0, NOISE - sum(p.shape), (pairs,)) per parameter
 *   - archive/10M/train/val/eggroll.py:122-128  direction d of parameter p = buffer[off_p[d] : off_p[d] + sum(shape)]
 * torch's CUDA Philox stream cannot be reproduced off an NVIDIA GPU, so the buffer and the offsets here are defined
 * by a counter-based generator; the slicing algebra above is kept exactly.
 *
 * Generator: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11).
 *   buffer value G[i], i < 2^28: out = philox(ctr = (i >> 2, 0, 0, STREAM_BUFFER), key = (seed_lo, seed_hi));
 *     Box-Muller on (out0, out1) gives lanes 0, 1 and on (out2, out3) lanes 2, 3; G[i] = lane i & 3.
 *   offset off_p[d] for step s: out = philox(ctr = (d, p, 0, STREAM_OFFSET), key = lo/hi of 1_000_003*seed + s);
 *     off = (out0 * range) >> 32 with range = 2^28 - sum(shape), i.e. an integer in [0, range).
 *   head-slab jitter (the replacement of train/val/dust.py:281's torch.randn): value d < 256 of draw g at token
 *     row r = lane d & 3 of Box-Muller on philox(ctr = (64 r + d / 4, g, 0, STREAM_HEAD), key = (seed_lo, seed_hi)).
 *   direct-draw jitter (the replacement of train/val/dust.py:244's torch.randn): channel d of a site `width` wide,
 *     draw g, site s, token row r = lane d & 3 of Box-Muller on philox(ctr = (r width / 4 + d / 4, g, s, STREAM_DUST),
 *     key = (seed_lo, seed_hi)).
 * Box-Muller: u1 = ((x >> 8) + 1) * 2^-24 in (0, 1], u2 = (y >> 8) * 2^-24 in [0, 1);
 *   r = sqrt(-2 ln u1), z0 = r cos(2 pi u2), z1 = r sin(2 pi u2).
 * ln, sin and cos are this file's own polynomials (atanh series for ln, Taylor series for sin/cos on [-pi/4, pi/4)
 * after an exact quadrant reduction), written with explicit fmaf and with floating-point contraction off, so that
 * the HIP kernels, which use the same operation sequence, reproduce every value bit for bit. sqrtf and the one
 * division are IEEE correctly rounded on both sides.
 *
 * Parity pins (tests/test_oracle_rng.py): Random123 known-answer vectors for Philox4x32-10, an independent numpy
 * Philox, libm (double) accuracy bounds for the polynomials, and normality statistics of the buffer.
 */
#include <math.h>
#include <stdint.h>

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u
#define STREAM_BUFFER 0x4E4F4953u /* "NOIS" */
#define STREAM_OFFSET 0x4F464653u /* "OFFS" */
#define STREAM_HEAD 0x44414548u   /* "HEAD" */
#define STREAM_DUST 0x54535544u   /* "DUST" */

void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int round = 0; round < 10; ++round) {
        uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* ln(u) for u in (0, 1]: u = m 2^e with m in (sqrt(1/2), sqrt(2)], ln m = 2 atanh(s), s = (m - 1) / (m + 1),
 * atanh(s) = s (1 + s^2/3 + s^4/5 + s^6/7 + s^8/9 + s^10/11); |s| <= 0.1716 so the dropped terms are < 1e-10. */
float oracle_ln(float u) {
    union { float f; uint32_t i; } v;
    v.f = u;
    int e = (int)((v.i >> 23) & 0xFF) - 127;
    v.i = (v.i & 0x007FFFFFu) | 0x3F800000u; /* m in [1, 2) */
    float m = v.f;
    if (m > 1.41421356f) { m = m * 0.5f; e = e + 1; }
    float s = (m - 1.0f) / (m + 1.0f);
    float z = s * s;
    float p = 1.0f / 11.0f;
    p = fmaf(p, z, 1.0f / 9.0f);
    p = fmaf(p, z, 1.0f / 7.0f);
    p = fmaf(p, z, 1.0f / 5.0f);
    p = fmaf(p, z, 1.0f / 3.0f);
    p = fmaf(p, z, 1.0f);
    float lnm = 2.0f * s * p;
    float fe = (float)e;
    /* ln 2 = LN2_HI + LN2_LO, LN2_HI with 16 significant bits so fe * LN2_HI is exact for |e| < 2^8 */
    const float LN2_HI = 0.693145751953125f, LN2_LO = 1.42860682030941723212e-6f;
    return fmaf(fe, LN2_HI, fmaf(fe, LN2_LO, lnm));
}

/* sin and cos of phi in [-pi/4, pi/4): Taylor polynomials through phi^9 and phi^10 (error < 3e-8). */
static void sincos_quarter(float phi, float* s, float* c) {
    float z = phi * phi;
    float ps = 1.0f / 362880.0f;
    ps = fmaf(ps, z, -1.0f / 5040.0f);
    ps = fmaf(ps, z, 1.0f / 120.0f);
    ps = fmaf(ps, z, -1.0f / 6.0f);
    ps = fmaf(ps, z, 1.0f);
    *s = phi * ps;
    float pc = -1.0f / 3628800.0f;
    pc = fmaf(pc, z, 1.0f / 40320.0f);
    pc = fmaf(pc, z, -1.0f / 720.0f);
    pc = fmaf(pc, z, 1.0f / 24.0f);
    pc = fmaf(pc, z, -0.5f);
    *c = fmaf(pc, z, 1.0f);
}

/* (cos, sin) of 2 pi u for u = k 2^-24 in [0, 1): 4u = q + f exactly, angle = q pi/2 + pi/4 + (f - 1/2) pi/2. */
void oracle_sincos2pi(float u, float* sn, float* cs) {
    float t = u * 4.0f;
    int q = (int)t;
    float f = t - (float)q;
    float phi = (f - 0.5f) * 1.57079632679489662f;
    float s, c;
    sincos_quarter(phi, &s, &c);
    const float R = 0.70710678118654752f;
    float c45 = (c - s) * R, s45 = (c + s) * R;
    switch (q) {
        case 0: *cs = c45; *sn = s45; break;
        case 1: *cs = -s45; *sn = c45; break;
        case 2: *cs = -c45; *sn = -s45; break;
        default: *cs = s45; *sn = -c45; break;
    }
}

void oracle_box_muller(uint32_t x, uint32_t y, float* z0, float* z1) {
    float u1 = (float)((x >> 8) + 1u) * 5.9604644775390625e-8f; /* 2^-24 */
    float u2 = (float)(y >> 8) * 5.9604644775390625e-8f;
    float r = sqrtf(-2.0f * oracle_ln(u1));
    float sn, cs;
    oracle_sincos2pi(u2, &sn, &cs);
    *z0 = r * cs;
    *z1 = r * sn;
}

/* n consecutive values G[start .. start + n) of the virtual Gaussian buffer. */
void oracle_noise_buffer(uint64_t seed, uint64_t start, int64_t n, float* out) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int64_t j = 0; j < n; ++j) {
        uint64_t i = start + (uint64_t)j;
        uint32_t ctr[4] = {(uint32_t)(i >> 2), 0u, 0u, STREAM_BUFFER};
        uint32_t r[4];
        float z[4];
        oracle_philox4x32_10(ctr, key, r);
        oracle_box_muller(r[0], r[1], &z[0], &z[1]);
        oracle_box_muller(r[2], r[3], &z[2], &z[3]);
        out[j] = z[i & 3];
    }
}

/* off_p[d] for directions d in [0, n): the offsets of one parameter at one step. */
void oracle_noise_offsets(uint64_t seed, uint64_t step, uint32_t param, uint32_t range, int64_t n, int64_t* out) {
    uint64_t s = 1000003ull * seed + step;
    uint32_t key[2] = {(uint32_t)s, (uint32_t)(s >> 32)};
    for (int64_t d = 0; d < n; ++d) {
        uint32_t ctr[4] = {(uint32_t)d, param, 0u, STREAM_OFFSET};
        uint32_t r[4];
        oracle_philox4x32_10(ctr, key, r);
        out[d] = (int64_t)(((uint64_t)r[0] * range) >> 32);
    }
}

/* rows[j, :] = G[off[j] : off[j] + width] for j < n: the gathered noise of n directions of one parameter. */
void oracle_noise_rows(uint64_t seed, const int64_t* off, int64_t n, int64_t width, float* rows) {
    for (int64_t j = 0; j < n; ++j) oracle_noise_buffer(seed, (uint64_t)off[j], width, rows + j * width);
}

/* out[i, d] = head-slab jitter of draw `draw` at rows row0 + i (i < n), d < 256. */
void oracle_head_noise(uint64_t seed, uint32_t draw, uint32_t row0, int64_t n, float* out) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int64_t i = 0; i < n; ++i)
        for (uint32_t q = 0; q < 64; ++q) {
            uint32_t ctr[4] = {((uint32_t)row0 + (uint32_t)i) * 64u + q, draw, 0u, STREAM_HEAD};
            uint32_t r[4];
            float* z = out + i * 256 + 4 * q;
            oracle_philox4x32_10(ctr, key, r);
            oracle_box_muller(r[0], r[1], &z[0], &z[1]);
            oracle_box_muller(r[2], r[3], &z[2], &z[3]);
        }
}

/* out[i, d] = direct-draw jitter of draw `draw` at site `site`, token rows row0 + i (i < n), d < width (% 4 == 0). */
void oracle_dust_noise(uint64_t seed, uint32_t draw, uint32_t site, uint32_t row0, int64_t n, int32_t width,
                       float* out) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    const uint32_t quads = (uint32_t)width / 4u;
    for (int64_t i = 0; i < n; ++i)
        for (uint32_t q = 0; q < quads; ++q) {
            uint32_t ctr[4] = {((uint32_t)row0 + (uint32_t)i) * quads + q, draw, site, STREAM_DUST};
            uint32_t r[4];
            float* z = out + i * width + 4 * q;
            oracle_philox4x32_10(ctr, key, r);
            oracle_box_muller(r[0], r[1], &z[0], &z[1]);
            oracle_box_muller(r[2], r[3], &z[2], &z[3]);
        }
}
