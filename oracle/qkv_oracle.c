/*
 * qkv_oracle.c -- CPU restatement of the reference's compressed-KV path.
 *
 * TEST INFRASTRUCTURE ONLY (see qkv_oracle.h).  Built with -ffp-contract=off
 * and without fast-math so every float operation rounds exactly once, in the
 * order the reference source writes it.
 *
 * Pinning (the independent check that fixes each function; tests/ file):
 *   or_f16_to_f32 / or_f32_to_f16   numpy float16 casts, exhaustive over all
 *                                   65536 halves + 2^20 random floats
 *                                   (test_oracle_codec.py)
 *   or_tq3_signs                    known answer: first 16 signs, 69 of 128
 *                                   positive, LE mask words 0xfae78245 ...
 *   or_tq3_centroids / bounds       bounds are centroid midpoints; centroids
 *                                   are the 8-level Gaussian Lloyd-Max levels
 *                                   times 1/sqrt(128)
 *   or_wht128                       Sylvester Hadamard matrix from
 *                                   scipy.linalg.hadamard, H*H = 128*I
 *   or_tq3_find_bin                 numpy.searchsorted(bounds, v, 'left') on
 *                                   random + all-boundary + signed-zero + NaN
 *   or_tq3_prescale_threshold_mismatches
 *                                   exhaustive over all 2^32 fp32 patterns; a
 *                                   threshold moved by one ulp must fail
 *   or_tq3_fold_mismatches          exhaustive over the reachable fp32
 *                                   patterns (both signs of the lane); a
 *                                   threshold moved by one ulp, or A = 2^24,
 *                                   must fail
 *   or_pack/unpack_3bit_8           numpy bit-level packing (LE 3-bit stream)
 *   or_tq3_encode                   fp64 rotation y = H*D*x/|x|/sqrt(128):
 *                                   codes equal searchsorted(bounds, y) except
 *                                   where |y - bound| < 4 ulp; norm equals the
 *                                   sequential fp32 sum (numpy cumsum) sqrt;
 *                                   zero-block rule
 *   or_tq3_decode                   fp64 D*H*c*norm/sqrt(128) within fp16 ulp
 *   or_q8_encode / decode           closed form: |x - q*d| <= d/2 (+fp16
 *                                   rounding of d), amax=0 -> d=+0 and q=0,
 *                                   ties to even, numpy rint cross-check
 *   or_attn_split + merge           or_attn_ref_f64 (softmax in double) for
 *                                   dense, causal-verify, tree, sink/window
 *                                   inputs; split-count invariance
 *   or_attn_ref_f64                 brute-force numpy softmax on tiny inputs
 *   or_attn_ref_f64_f32kv           equals or_attn_ref_f64 bit for bit on
 *                                   fp16-representable float inputs (same core)
 * No function is "parity unpinned".
 */
#include "qkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ===================================================================== */
/* fp16 <-> fp32 (IEEE binary16, round-to-nearest-even)                   */
/* ===================================================================== */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: value = man * 2^-24, exact in fp32 */
        float v = (float)man * bits_f32(0x33800000u); /* 2^-24 */
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {                       /* inf / nan */
        if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (a >= 0x38800000u) {                       /* normal half range */
        uint32_t exp = (a >> 23) - 112u;
        uint32_t man = a & 0x7fffffu;
        uint32_t h = (exp << 10) | (man >> 13);
        uint32_t rem = man & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    /* subnormal or zero in half: value / 2^-24 rounded to even integer */
    {
        float v = bits_f32(a) * bits_f32(0x4b800000u); /* * 2^24 (exact) */
        /* v < 1024; round half to even */
        float fl = floorf(v);
        float r = v - fl;
        uint32_t q = (uint32_t)fl;
        if (r > 0.5f || (r == 0.5f && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
}

void or_f16_to_f32_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = or_f16_to_f32(h[i]);
}
void or_f32_to_f16_n(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = or_f32_to_f16(f[i]);
}

/* ===================================================================== */
/* Codec constants                                                         */
/* ===================================================================== */

/* turboquant.cuh:27-30 (data, kept identical) */
static const float k_centroids[8] = {
    -0.190303f, -0.118828f, -0.066847f, -0.021664f,
     0.021664f,  0.066847f,  0.118828f,  0.190303f};
/* turboquant.cuh:34-37 (data, kept identical) */
static const float k_bounds[7] = {
    -0.154566f, -0.092838f, -0.044256f, 0.000000f,
     0.044256f,  0.092838f,  0.154566f};

void or_tq3_centroids(float out[8]) { memcpy(out, k_centroids, sizeof(k_centroids)); }
void or_tq3_bounds(float out[7]) { memcpy(out, k_bounds, sizeof(k_bounds)); }

/* turboquant.cuh:61 rsqrtf(128.0f).  The correctly rounded value of
 * 1/sqrt(128) is used (0x3DB504F3). */
float or_tq3_wht_scale(void) { return bits_f32(0x3DB504F3u); }

/* turboquant.cuh:288-302: xorshift64 from 0xCAFEF00D, bit 0 picks the sign. */
void or_tq3_signs(float out[OR_TQ_BLOCK]) {
    uint64_t s = 0xCAFEF00DULL;
    for (int i = 0; i < OR_TQ_BLOCK; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = (s & 1u) ? 1.0f : -1.0f;
    }
}

static float g_signs[OR_TQ_BLOCK];
static int g_signs_ready = 0;
static const float* signs(void) {
    if (!g_signs_ready) { or_tq3_signs(g_signs); g_signs_ready = 1; }
    return g_signs;
}

/* ===================================================================== */
/* Building blocks                                                         */
/* ===================================================================== */

/* turboquant.cuh:48-64: in-place Sylvester butterflies, strides 1..64,
 * (a,b) -> (a+b, a-b), then every element times rsqrtf(128). */
void or_wht128(float* x) {
    for (int step = 1; step < OR_TQ_BLOCK; step <<= 1)
        for (int i = 0; i < OR_TQ_BLOCK; i += 2 * step)
            for (int j = i; j < i + step; j++) {
                float a = x[j], b = x[j + step];
                x[j] = a + b;
                x[j + step] = a - b;
            }
    const float rs = or_tq3_wht_scale();
    for (int i = 0; i < OR_TQ_BLOCK; i++) x[i] *= rs;
}

/* turboquant.cuh:79-87: idx = number of bounds strictly below v. */
uint8_t or_tq3_find_bin(float v) {
    uint8_t idx = 0;
    for (int i = 0; i < 7; i++)
        if (v > k_bounds[i]) idx = (uint8_t)(i + 1);
    return idx;
}

/* Check of a table of bin thresholds on the WHT output before the x rs
 * scaling (the form the GPU encoder uses): for every fp32 bit pattern w in
 * [lo, hi], or_tq3_find_bin(fl(w * rs)) must equal #{k : w > thr[k]}.  With
 * `negated`, the pattern holds v = -w (a lane that carries its butterfly
 * output negated) and the bin of w must equal 7 - #{k : v > thr[k]} (NaN
 * patterns skipped).  Returns the number of bit patterns where the two
 * differ; over [0, 2^32 - 1] a zero proves the folding exact. */
int64_t or_tq3_prescale_threshold_mismatches(const uint32_t* thr, int64_t lo, int64_t hi,
                                             int negated, int nthreads) {
    const float rs = or_tq3_wht_scale();
    float t[7];
    for (int k = 0; k < 7; k++) t[k] = bits_f32(thr[k]);
    int64_t bad = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads) reduction(+ : bad)
#endif
    for (int64_t u = lo; u <= hi; u++) {
        const float v = bits_f32((uint32_t)u);
        uint8_t c = 0;
        for (int k = 0; k < 7; k++) c = (uint8_t)(c + (v > t[k]));
        if (!negated) {
            bad += (c != or_tq3_find_bin(v * rs));
        } else if (v == v) {
            /* v holds -w: the bin of w is 7 minus the count (NaN is excluded:
             * a NaN element only occurs in a block with a non-finite norm,
             * whose codes are zero by rule) */
            const float w = -v;
            bad += ((uint8_t)(7 - c) != or_tq3_find_bin(w * rs));
        }
    }
    return bad;
}

/* Check of the sign-folded binning (the GPU encoder's form): with
 * y = fl(-A w + |w|) (one rounding; exact in double before the float cast),
 * bin(w) must equal 4 + m for signbit(y) = 1 and 3 - m otherwise, with
 * m = #{j : |y| > q[j]}.  With `negated` the pattern holds v = -w and
 * y = fl(A v + |v|).  Checked patterns: w = +-0 and 2^-67 <= |w| < 2^100 (the
 * reachable WHT outputs: every nonzero one is a multiple of 2^-67).  Returns
 * the number of mismatching bit patterns in [lo, hi]. */
int64_t or_tq3_fold_mismatches(uint32_t a_bits, const uint32_t* q, int64_t lo, int64_t hi,
                               int negated, int nthreads) {
    const float rs = or_tq3_wht_scale();
    const double A = (double)bits_f32(a_bits);
    float t[3];
    for (int k = 0; k < 3; k++) t[k] = bits_f32(q[k]);
    int64_t bad = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads) reduction(+ : bad)
#endif
    for (int64_t u = lo; u <= hi; u++) {
        const uint32_t e = ((uint32_t)u >> 23) & 0xffu;
        if ((((uint32_t)u & 0x7fffffffu) != 0u) && (e < 127u - 67u || e >= 127u + 100u)) continue;
        const float v = bits_f32((uint32_t)u);
        const double dv = (double)v;
        const float y = (float)((negated ? A : -A) * dv + fabs(dv));
        uint32_t ybits;
        memcpy(&ybits, &y, 4);
        const float ay = fabsf(y);
        const int m = (ay > t[0]) + (ay > t[1]) + (ay > t[2]);
        const int idx = (ybits >> 31) ? 4 + m : 3 - m;
        const float w = negated ? -v : v;
        bad += ((uint8_t)idx != or_tq3_find_bin(w * rs));
    }
    return bad;
}

/* turboquant.cuh:90-100 */
void or_pack_3bit_8(uint8_t* dst, const uint8_t* idx8) {
    uint32_t p = 0;
    for (int i = 0; i < 8; i++) p |= ((uint32_t)idx8[i]) << (3 * i);
    dst[0] = (uint8_t)(p & 0xff);
    dst[1] = (uint8_t)((p >> 8) & 0xff);
    dst[2] = (uint8_t)((p >> 16) & 0xff);
}

/* turboquant.cuh:103-108 */
void or_unpack_3bit_8(const uint8_t* src, uint8_t* idx8) {
    uint32_t p = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16);
    for (int i = 0; i < 8; i++) idx8[i] = (uint8_t)((p >> (3 * i)) & 7u);
}

/* ===================================================================== */
/* TQ3 encode / decode                                                     */
/* ===================================================================== */

/* turboquant.cuh:112-165, one block. */
static void tq3_encode_one(const uint16_t* in, or_block_tq3* out, float* rot_out) {
    const float* sg = signs();
    float x[OR_TQ_BLOCK];
    for (int i = 0; i < OR_TQ_BLOCK; i++) x[i] = or_f16_to_f32(in[i]);
    float nsq = 0.0f;
    for (int i = 0; i < OR_TQ_BLOCK; i++) nsq += x[i] * x[i];
    float norm = sqrtf(nsq);
    out->norm = norm;
    if (norm < 1e-10f) {
        memset(out->qs, 0, OR_TQ_QS_BYTES);
        if (rot_out) memset(rot_out, 0, sizeof(float) * OR_TQ_BLOCK);
        return;
    }
    float inv = 1.0f / norm;
    for (int i = 0; i < OR_TQ_BLOCK; i++) x[i] *= inv;
    for (int i = 0; i < OR_TQ_BLOCK; i++) x[i] *= sg[i];
    or_wht128(x);
    uint8_t idx[OR_TQ_BLOCK];
    for (int i = 0; i < OR_TQ_BLOCK; i++) idx[i] = or_tq3_find_bin(x[i]);
    for (int g = 0; g < OR_TQ_BLOCK / 8; g++) or_pack_3bit_8(&out->qs[3 * g], &idx[8 * g]);
    if (rot_out) memcpy(rot_out, x, sizeof(float) * OR_TQ_BLOCK);
}

void or_tq3_encode(const uint16_t* in_f16, or_block_tq3* out, int64_t n_blocks, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t b = 0; b < n_blocks; b++)
        tq3_encode_one(in_f16 + b * OR_TQ_BLOCK, out + b, NULL);
    (void)nthreads;
}

void or_tq3_encode_rotated(const uint16_t* in_f16, or_block_tq3* out, float* rot,
                           int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++)
        tq3_encode_one(in_f16 + b * OR_TQ_BLOCK, out + b, rot + b * OR_TQ_BLOCK);
}

/* turboquant.cuh:169-200 (and 253-284 when out_f32 != NULL). */
static void tq3_decode_one(const or_block_tq3* in, uint16_t* out_f16, float* out_f32) {
    const float* sg = signs();
    float norm = in->norm;
    float x[OR_TQ_BLOCK];
    for (int g = 0; g < OR_TQ_BLOCK / 8; g++) {
        uint8_t idx[8];
        or_unpack_3bit_8(&in->qs[3 * g], idx);
        for (int j = 0; j < 8; j++) x[8 * g + j] = k_centroids[idx[j]];
    }
    or_wht128(x);
    for (int i = 0; i < OR_TQ_BLOCK; i++) x[i] *= sg[i];
    for (int i = 0; i < OR_TQ_BLOCK; i++) {
        float v = x[i] * norm;
        if (out_f16) out_f16[i] = or_f32_to_f16(v);
        if (out_f32) out_f32[i] = v;
    }
}

void or_tq3_decode(const or_block_tq3* in, uint16_t* out_f16, int64_t n_blocks, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t b = 0; b < n_blocks; b++)
        tq3_decode_one(in + b, out_f16 + b * OR_TQ_BLOCK, NULL);
    (void)nthreads;
}

void or_tq3_decode_f32(const or_block_tq3* in, float* out, int64_t n_blocks) {
    for (int64_t b = 0; b < n_blocks; b++) tq3_decode_one(in + b, NULL, out + b * OR_TQ_BLOCK);
}

/* ===================================================================== */
/* Q8_0 KV                                                                 */
/* ===================================================================== */

/* __float2int_rn: round half to even; NaN -> 0 (saturating convert). */
static int f2i_rn(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int)0x80000000u;
    return (int)nearbyintf(v); /* default rounding mode: to nearest even */
}

/* attention.cuh:2587-2609, one block (pad is not written). */
static void q8_encode_one(const uint16_t* in, or_block_q8* out) {
    float v[OR_Q8_BLOCK];
    float amax = 0.0f;
    for (int i = 0; i < OR_Q8_BLOCK; i++) v[i] = or_f16_to_f32(in[i]);
    /* fmaxf reduction over |v| (order is irrelevant for max; fmaxf drops NaN) */
    amax = fabsf(v[0]);
    for (int i = 1; i < OR_Q8_BLOCK; i++) amax = fmaxf(amax, fabsf(v[i]));
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    for (int i = 0; i < OR_Q8_BLOCK; i++) {
        int q = f2i_rn(v[i] * inv);
        if (q > 127) q = 127;
        if (q < -128) q = -128;
        out->qs[i] = (int8_t)q;
    }
    out->d = or_f32_to_f16(scale);
}

void or_q8_encode(const uint16_t* in_f16, or_block_q8* out, int64_t n_blocks, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t b = 0; b < n_blocks; b++) q8_encode_one(in_f16 + b * OR_Q8_BLOCK, out + b);
    (void)nthreads;
}

/* attention.cuh:2614-2626 */
void or_q8_decode(const or_block_q8* in, uint16_t* out_f16, int64_t n_blocks, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t b = 0; b < n_blocks; b++) {
        float s = or_f16_to_f32(in[b].d);
        for (int i = 0; i < OR_Q8_BLOCK; i++)
            out_f16[b * OR_Q8_BLOCK + i] = or_f32_to_f16((float)in[b].qs[i] * s);
    }
    (void)nthreads;
}

/* ===================================================================== */
/* Split-K flash decode                                                    */
/* ===================================================================== */

#define OR_BM 32

int or_key_visible(int key, int start_pos, int t_idx, int sink_tok, int window_tok,
                   const uint32_t* tree_mask) {
    int active_end_t = start_pos + t_idx + 1;               /* attention.cuh:1941-1942 */
    if (key < 0 || key >= active_end_t) return 0;
    if (sink_tok > 0 || window_tok > 0) {                   /* attention.cuh:1983-1994 */
        int ts = key & ~(OR_BM - 1);
        int te = ts + OR_BM < active_end_t ? ts + OR_BM : active_end_t;
        int win_lo = active_end_t - window_tok;
        if (!(ts < sink_tok) && !(te > win_lo)) return 0;
    }
    if (tree_mask && key >= start_pos)                      /* attention.cuh:2101-2105 */
        return (int)((tree_mask[t_idx] >> (key - start_pos)) & 1u);
    return 1;
}

/* Decode one key or value row of one kv head into fp16 (the reference's smem
 * tile contents): TQ3 per attention.cuh:2009-2072, Q8 per attention.cuh:2720-2729. */
static void decode_row(int kind, const void* cache, int pos, int num_kv, int kv_head, int hd,
                       uint16_t* dst) {
    if (kind == OR_KV_TQ3) {
        int bpk = hd / OR_TQ_BLOCK;
        const or_block_tq3* b = (const or_block_tq3*)cache + ((int64_t)pos * num_kv + kv_head) * bpk;
        for (int j = 0; j < bpk; j++) tq3_decode_one(b + j, dst + j * OR_TQ_BLOCK, NULL);
    } else if (kind == OR_KV_Q8) {
        int bpk = hd / OR_Q8_BLOCK;
        const or_block_q8* b = (const or_block_q8*)cache + ((int64_t)pos * num_kv + kv_head) * bpk;
        for (int j = 0; j < bpk; j++) {
            float s = or_f16_to_f32(b[j].d);
            for (int i = 0; i < OR_Q8_BLOCK; i++)
                dst[j * OR_Q8_BLOCK + i] = or_f32_to_f16((float)b[j].qs[i] * s);
        }
    } else {
        const uint16_t* src = (const uint16_t*)cache + ((int64_t)pos * num_kv + kv_head) * hd;
        memcpy(dst, src, sizeof(uint16_t) * hd);
    }
}

/* Score of one (q head, key row): the reference splits the HD-long dot product
 * over 32 lanes (LANE_D = HD/32 consecutive elements each, accumulated as
 * half2 pairs) and reduces with an xor butterfly (attention.cuh:2081-2095);
 * this reproduces that association (lane 0's view of the butterfly). */
static float score_dot(const float* qf, const float* kf, int hd) {
    float part[32];
    int lane_d = hd / 32;
    for (int lane = 0; lane < 32; lane++) {
        float p = 0.0f;
        for (int i = 0; i < lane_d / 2; i++) {
            int c = lane * lane_d + 2 * i;
            p += qf[c] * kf[c] + qf[c + 1] * kf[c + 1];
        }
        part[lane] = p;
    }
    for (int off = 16; off > 0; off >>= 1) {
        float nxt[32];
        for (int lane = 0; lane < 32; lane++) nxt[lane] = part[lane] + part[lane ^ off];
        memcpy(part, nxt, sizeof(part));
    }
    return part[0];
}

/* Online-softmax state of one (kv_head, t_idx, split): gqa rows. */
typedef struct {
    float* qf;     /* [gqa][hd] query */
    float* acc;    /* [gqa][hd] unnormalized output */
    float* m;      /* [gqa] running max */
    float* l;      /* [gqa] running sum */
    uint16_t* krow; uint16_t* vrow;   /* [OR_BM][hd] tile rows (fp16) */
    float* kf; float* vf;             /* [OR_BM][hd] as floats */
} split_state;

static void split_state_init(split_state* st, const uint16_t* q, int num_q, int num_kv, int hd,
                             int kv_head, int t_idx) {
    const int gqa = num_q / num_kv;
    st->qf = (float*)malloc(sizeof(float) * gqa * hd);
    st->acc = (float*)calloc((size_t)gqa * hd, sizeof(float));
    st->m = (float*)malloc(sizeof(float) * gqa);
    st->l = (float*)calloc(gqa, sizeof(float));
    st->krow = (uint16_t*)malloc(sizeof(uint16_t) * OR_BM * hd);
    st->vrow = (uint16_t*)malloc(sizeof(uint16_t) * OR_BM * hd);
    st->kf = (float*)malloc(sizeof(float) * OR_BM * hd);
    st->vf = (float*)malloc(sizeof(float) * OR_BM * hd);
    for (int g = 0; g < gqa; g++) {
        st->m[g] = -INFINITY;
        int qh = kv_head * gqa + g;
        for (int c = 0; c < hd; c++)
            st->qf[g * hd + c] = or_f16_to_f32(q[((int64_t)t_idx * num_q + qh) * hd + c]);
    }
}

static void split_state_store(split_state* st, float* part_m, float* part_l, float* part_o,
                              int num_q, int num_kv, int hd, int sub_n_max, int k_splits,
                              int kv_head, int t_idx, int split) {
    const int gqa = num_q / num_kv;
    for (int g = 0; g < gqa; g++) {
        int qh = kv_head * gqa + g;
        int64_t ml = ((int64_t)qh * sub_n_max + t_idx) * k_splits + split;
        part_m[ml] = st->m[g];
        part_l[ml] = st->l[g];
        memcpy(part_o + ml * hd, st->acc + g * hd, sizeof(float) * hd);
    }
    free(st->qf); free(st->acc); free(st->m); free(st->l);
    free(st->krow); free(st->vrow); free(st->kf); free(st->vf);
}

/* One BM = 32 key tile [ts, ts + len) of the split kernels' loop body
 * (attention.cuh:2009-2150): decode to fp16, scores (score_dot) * scale with
 * invisible keys -inf (key >= start_pos and its tree bit clear), online
 * softmax with expf, the xor-butterfly sum of p, sequential acc += p * v. */
static void split_tile(split_state* st, int kind, const void* k, const void* v, int num_kv,
                       int hd, int gqa, int start_pos, float scale, const uint32_t* tree_mask,
                       int kv_head, int t_idx, int ts, int len) {
    float s[OR_BM], p[OR_BM];
    for (int r = 0; r < len; r++) {
        decode_row(kind, k, ts + r, num_kv, kv_head, hd, st->krow + r * hd);
        decode_row(kind, v, ts + r, num_kv, kv_head, hd, st->vrow + r * hd);
    }
    for (int i = 0; i < len * hd; i++) {
        st->kf[i] = or_f16_to_f32(st->krow[i]);
        st->vf[i] = or_f16_to_f32(st->vrow[i]);
    }
    for (int g = 0; g < gqa; g++) {
        float mrow = -INFINITY;
        for (int r = 0; r < OR_BM; r++) {
            float val = -INFINITY;
            if (r < len) {
                int key = ts + r;
                int vis = (key < start_pos) ||
                          (tree_mask ? (int)((tree_mask[t_idx] >> (key - start_pos)) & 1u) : 1);
                if (vis) val = score_dot(st->qf + g * hd, st->kf + r * hd, hd) * scale;
            }
            s[r] = val;
            mrow = fmaxf(mrow, val);
        }
        float mnew = fmaxf(st->m[g], mrow);
        float corr = expf(st->m[g] - mnew);
        float sum = 0.0f;
        for (int r = 0; r < OR_BM; r++) { p[r] = expf(s[r] - mnew); }
        /* xor-butterfly sum over 32 lanes (attention.cuh:2121-2123) */
        {
            float part[32];
            for (int r = 0; r < 32; r++) part[r] = r < OR_BM ? p[r] : 0.0f;
            for (int off = 16; off > 0; off >>= 1) {
                float nxt[32];
                for (int r = 0; r < 32; r++) nxt[r] = part[r] + part[r ^ off];
                memcpy(part, nxt, sizeof(part));
            }
            sum = part[0];
        }
        for (int c = 0; c < hd; c++) st->acc[g * hd + c] *= corr;
        st->l[g] = st->l[g] * corr + sum;
        for (int r = 0; r < len; r++)
            for (int c = 0; c < hd; c++) st->acc[g * hd + c] += p[r] * st->vf[r * hd + c];
        st->m[g] = mnew;
    }
}

/* attention.cuh:1905-2177 / 2633-2801 for one (kv_head, t_idx, split). */
static void split_one(int kind, const uint16_t* q, const void* k, const void* v,
                      float* part_m, float* part_l, float* part_o, int num_q, int num_kv,
                      int hd, int start_pos, int sub_n_max, int active_end_max, float scale,
                      int k_splits, int sink_tok, int window_tok, const uint32_t* tree_mask,
                      int kv_head, int t_idx, int split) {
    const int gqa = num_q / num_kv;
    const int abs_pos = start_pos + t_idx;
    const int active_end_t = abs_pos + 1;
    const int total_tiles = (active_end_max + OR_BM - 1) / OR_BM;
    const int tps = (total_tiles + k_splits - 1) / k_splits;
    const int tile_lo = split * tps * OR_BM;
    int tile_hi = (split + 1) * tps * OR_BM;
    if (tile_hi > active_end_t) tile_hi = active_end_t;

    split_state st;
    split_state_init(&st, q, num_q, num_kv, hd, kv_head, t_idx);
    const int sparse = (sink_tok > 0 || window_tok > 0);
    const int win_lo = sparse ? active_end_t - window_tok : 0;
    for (int ts = tile_lo; ts < tile_hi; ts += OR_BM) {
        int te = ts + OR_BM < tile_hi ? ts + OR_BM : tile_hi;
        int len = te - ts;
        if (sparse && !(ts < sink_tok) && !(te > win_lo)) continue;
        split_tile(&st, kind, k, v, num_kv, hd, gqa, start_pos, scale, tree_mask, kv_head, t_idx,
                   ts, len);
    }
    split_state_store(&st, part_m, part_l, part_o, num_q, num_kv, hd, sub_n_max, k_splits,
                      kv_head, t_idx, split);
}

void or_attn_split(int kind, const uint16_t* q, const void* k, const void* v,
                   float* part_m, float* part_l, float* part_o,
                   int num_q, int num_kv, int hd, int start_pos, int sub_n,
                   int sub_n_max, int active_end_max, float scale, int k_splits,
                   int sink_tok, int window_tok, const uint32_t* tree_mask,
                   int nthreads) {
    int64_t n_items = (int64_t)num_kv * sub_n * k_splits;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic) num_threads(nthreads)
#endif
    for (int64_t it = 0; it < n_items; it++) {
        int split = (int)(it % k_splits);
        int t_idx = (int)((it / k_splits) % sub_n);
        int kv_head = (int)(it / ((int64_t)k_splits * sub_n));
        split_one(kind, q, k, v, part_m, part_l, part_o, num_q, num_kv, hd, start_pos,
                  sub_n_max, active_end_max, scale, k_splits, sink_tok, window_tok,
                  tree_mask, kv_head, t_idx, split);
    }
    (void)nthreads;
}

/* attention.cuh:1837-1891 */
void or_attn_split_merge(const float* part_m, const float* part_l, const float* part_o,
                         uint16_t* out, int num_q, int num_kv, int hd, int sub_n,
                         int sub_n_max, int k_splits) {
    (void)num_kv;
    float* o = (float*)malloc(sizeof(float) * hd);
    for (int t = 0; t < sub_n; t++)
        for (int qh = 0; qh < num_q; qh++) {
            int64_t base = ((int64_t)qh * sub_n_max + t) * k_splits;
            float mg = -INFINITY;
            for (int s = 0; s < k_splits; s++) mg = fmaxf(mg, part_m[base + s]);
            float lg = 0.0f;
            for (int c = 0; c < hd; c++) o[c] = 0.0f;
            for (int s = 0; s < k_splits; s++) {
                float ms = part_m[base + s], ls = part_l[base + s];
                if (!isfinite(ms) || ls <= 0.0f) continue;
                float w = expf(ms - mg);
                lg += w * ls;
                const float* op = part_o + (base + s) * hd;
                for (int c = 0; c < hd; c++) o[c] += w * op[c];
            }
            float inv = lg > 0.0f ? 1.0f / lg : 0.0f;
            for (int c = 0; c < hd; c++)
                out[((int64_t)t * num_q + qh) * hd + c] = or_f32_to_f16(o[c] * inv);
        }
    free(o);
}

/* Independent fp64 reference (tools/dflash_attn_bench.cu:185-211 pattern). */
/* fp64 attention of query t over keys 0 .. start_pos + t that pass the
 * visibility rule; K/V elements are fp16 bits (kv_f32 = 0) or floats
 * (kv_f32 = 1: e.g. the exact, unrounded TQ3 dequantization).  Parallel over
 * (query, q head); each output row is a plain softmax in double. */
static void attn_ref_f64_any(const uint16_t* q, const void* k, const void* v, int kv_f32,
                             double* out, int num_q, int num_kv, int hd, int start_pos,
                             int sub_n, double scale, int sink_tok, int window_tok,
                             const uint32_t* tree_mask) {
    const int gqa = num_q / num_kv;
    #pragma omp parallel for collapse(2) schedule(dynamic)
    for (int t = 0; t < sub_n; t++) {
        for (int qh = 0; qh < num_q; qh++) {
            const int n_keys = start_pos + t + 1;
            double* sc = (double*)malloc(sizeof(double) * (n_keys > 0 ? n_keys : 1));
            const int kvh = qh / gqa;
            const uint16_t* qv = q + ((int64_t)t * num_q + qh) * hd;
            double mx = -INFINITY;
            for (int key = 0; key < n_keys; key++) {
                if (!or_key_visible(key, start_pos, t, sink_tok, window_tok, tree_mask)) {
                    sc[key] = -INFINITY;
                    continue;
                }
                const int64_t kr = ((int64_t)key * num_kv + kvh) * hd;
                double d = 0.0;
                for (int c = 0; c < hd; c++) {
                    const double kc = kv_f32 ? (double)((const float*)k)[kr + c]
                                             : (double)or_f16_to_f32(((const uint16_t*)k)[kr + c]);
                    d += (double)or_f16_to_f32(qv[c]) * kc;
                }
                sc[key] = d * scale;
                if (sc[key] > mx) mx = sc[key];
            }
            double den = 0.0;
            double* o = out + ((int64_t)t * num_q + qh) * hd;
            for (int c = 0; c < hd; c++) o[c] = 0.0;
            if (mx != -INFINITY) {
                for (int key = 0; key < n_keys; key++) {
                    if (sc[key] == -INFINITY) continue;
                    double w = exp(sc[key] - mx);
                    den += w;
                    const int64_t vr = ((int64_t)key * num_kv + kvh) * hd;
                    for (int c = 0; c < hd; c++)
                        o[c] += w * (kv_f32 ? (double)((const float*)v)[vr + c]
                                            : (double)or_f16_to_f32(((const uint16_t*)v)[vr + c]));
                }
                for (int c = 0; c < hd; c++) o[c] /= den;
            }
            free(sc);
        }
    }
}

void or_attn_ref_f64(const uint16_t* q, const uint16_t* k_f16, const uint16_t* v_f16,
                     double* out, int num_q, int num_kv, int hd, int start_pos,
                     int sub_n, double scale, int sink_tok, int window_tok,
                     const uint32_t* tree_mask) {
    attn_ref_f64_any(q, k_f16, v_f16, 0, out, num_q, num_kv, hd, start_pos, sub_n, scale,
                     sink_tok, window_tok, tree_mask);
}

void or_attn_ref_f64_f32kv(const uint16_t* q, const float* k, const float* v, double* out,
                           int num_q, int num_kv, int hd, int start_pos, int sub_n, double scale,
                           int sink_tok, int window_tok, const uint32_t* tree_mask) {
    attn_ref_f64_any(q, k, v, 1, out, num_q, num_kv, hd, start_pos, sub_n, scale, sink_tok,
                     window_tok, tree_mask);
}

/* ===================================================================== */
/* Legacy short-context decode (model.cuh:2544-2664)                      */
/* ===================================================================== */
/* Below 4096 cache rows the reference decodes one query token without the
 * fused split kernel: the keys (and later the values) are dequantized to an
 * fp16 scratch, then attn_score_kernel_h, softmax_kernel and
 * attn_value_kernel_h run over all seq_len rows (every row visible).  With
 * TQ_FUSED set, TQ3 keys / values go through attn_score_kernel_tq3 /
 * attn_value_kernel_tq3 instead, which dequantize to fp32 without the fp16
 * rounding.  `sum += a * b` in these kernels is taken as contracted to one
 * fused multiply-add (nvcc's default -fmad=true); fmaf states it here. */

/* lane 0's value after `for (off = 16; off > 0; off >>= 1) x += shfl_xor(x, off)`
 * over 32 lanes (attention.cuh:300-301) */
static float warp_butterfly_lane0(const float* x32) {
    float part[32];
    memcpy(part, x32, sizeof(part));
    for (int off = 16; off > 0; off >>= 1) {
        float nxt[32];
        for (int l = 0; l < 32; l++) nxt[l] = part[l] + part[l ^ off];
        memcpy(part, nxt, sizeof(part));
    }
    return part[0];
}

/* block-wide sum of per-thread values v[0..bd) (bd a multiple of 32): per
 * warp the butterfly, then warp 0 reduces the warp sums, lanes at or above
 * n_warps contributing 0 (attention.cuh:300-314) */
static float block_sum_legacy(const float* v, int bd) {
    const int n_warps = bd / 32;
    float ws[32];
    for (int l = 0; l < 32; l++) ws[l] = 0.0f;
    for (int w = 0; w < n_warps; w++) ws[w] = warp_butterfly_lane0(v + 32 * w);
    return warp_butterfly_lane0(ws);
}

/* attn_score_kernel_h (attention.cuh:277-316): blockDim = min(hd, 256), thread
 * t sums elements t, t + blockDim, ...; score = sum * scale. */
static void legacy_scores_h(const uint16_t* q, const uint16_t* k16, float* scores, int num_q,
                            int num_kv, int hd, int seq_len, float scale) {
    const int bd = hd < 256 ? hd : 256;
    const int gqa = num_q / num_kv;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int qh = 0; qh < num_q; qh++) {
        for (int pos = 0; pos < seq_len; pos++) {
            float th[256];
            const uint16_t* qv = q + (int64_t)qh * hd;
            const uint16_t* kv = k16 + ((int64_t)pos * num_kv + qh / gqa) * hd;
            for (int t = 0; t < bd; t++) {
                float s = 0.0f;
                for (int i = t; i < hd; i += bd)
                    s = fmaf(or_f16_to_f32(qv[i]), or_f16_to_f32(kv[i]), s);
                th[t] = s;
            }
            scores[(int64_t)qh * seq_len + pos] = block_sum_legacy(th, bd) * scale;
        }
    }
}

/* One TQ3 block dequantized as attn_score_kernel_tq3 / attn_value_kernel_tq3
 * do (attention.cuh:420-445, 941-963): centroids, the butterflies, then
 * x * (sign * (rsqrtf(128) * norm)), fp32, no fp16 rounding. */
static void legacy_tq3_block_f32(const or_block_tq3* b, float* x) {
    const float* sg = signs();
    for (int g = 0; g < OR_TQ_BLOCK / 8; g++) {
        uint8_t idx[8];
        or_unpack_3bit_8(&b->qs[3 * g], idx);
        for (int j = 0; j < 8; j++) x[8 * g + j] = k_centroids[idx[j]];
    }
    for (int step = 1; step < OR_TQ_BLOCK; step <<= 1)
        for (int i = 0; i < OR_TQ_BLOCK; i += 2 * step)
            for (int j = i; j < i + step; j++) {
                const float a = x[j], c = x[j + step];
                x[j] = a + c;
                x[j + step] = a - c;
            }
    const float scale_norm = or_tq3_wht_scale() * b->norm;
    for (int i = 0; i < OR_TQ_BLOCK; i++) x[i] *= sg[i] * scale_norm;
}

/* attn_score_kernel_tq3 (attention.cuh:400-483): blockDim = hd, thread t holds
 * K element t; prod = fp16(q_t) * k_t, reduced as above, times scale. */
static void legacy_scores_tq3(const uint16_t* q, const or_block_tq3* k, float* scores, int num_q,
                              int num_kv, int hd, int seq_len, float scale) {
    const int gqa = num_q / num_kv, bpk = hd / OR_TQ_BLOCK;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int kvh = 0; kvh < num_kv; kvh++) {
        for (int pos = 0; pos < seq_len; pos++) {
            float kx[512], th[512];
            for (int j = 0; j < bpk; j++)
                legacy_tq3_block_f32(k + ((int64_t)pos * num_kv + kvh) * bpk + j,
                                     kx + j * OR_TQ_BLOCK);
            for (int qi = 0; qi < gqa; qi++) {
                const int qh = kvh * gqa + qi;
                for (int t = 0; t < hd; t++) th[t] = or_f16_to_f32(q[(int64_t)qh * hd + t]) * kx[t];
                scores[(int64_t)qh * seq_len + pos] = block_sum_legacy(th, hd) * scale;
            }
        }
    }
}

/* softmax_kernel (attention.cuh:531-575) with st threads, st the least power
 * of two >= min(seq_len, 256): max, e = expf(x - max), per-thread strided
 * sums, a shared-memory tree, row *= 1 / (sum + 1e-10). */
static void legacy_softmax(float* scores, int num_q, int seq_len) {
    int st = 1;
    while (st < seq_len && st < 256) st <<= 1;
    for (int qh = 0; qh < num_q; qh++) {
        float* row = scores + (int64_t)qh * seq_len;
        float mx = -1e30f;
        for (int i = 0; i < seq_len; i++) mx = fmaxf(mx, row[i]);
        float sd[256];
        for (int t = 0; t < st; t++) {
            float s = 0.0f;
            for (int i = t; i < seq_len; i += st) {
                const float e = expf(row[i] - mx);
                row[i] = e;
                s += e;
            }
            sd[t] = s;
        }
        for (int s = st / 2; s > 0; s >>= 1)
            for (int t = 0; t < s; t++) sd[t] += sd[t + s];
        const float inv = 1.0f / (sd[0] + 1e-10f);
        for (int i = 0; i < seq_len; i++) row[i] *= inv;
    }
}

/* attn_value_kernel_h (attention.cuh:885-907): out[d] = fp16(sequential sum
 * over pos of p * v). */
static void legacy_values_h(const float* probs, const uint16_t* v16, uint16_t* out, int num_q,
                            int num_kv, int hd, int seq_len) {
    const int gqa = num_q / num_kv;
    #pragma omp parallel for schedule(static)
    for (int qh = 0; qh < num_q; qh++) {
        const float* sc = probs + (int64_t)qh * seq_len;
        for (int d = 0; d < hd; d++) {
            float s = 0.0f;
            for (int pos = 0; pos < seq_len; pos++)
                s = fmaf(sc[pos], or_f16_to_f32(v16[((int64_t)pos * num_kv + qh / gqa) * hd + d]), s);
            out[(int64_t)qh * hd + d] = or_f32_to_f16(s);
        }
    }
}

/* attn_value_kernel_tq3 (attention.cuh:920-989): per (kv head, 128-dim
 * block), acc += p * v over pos with v dequantized in fp32. */
static void legacy_values_tq3(const float* probs, const or_block_tq3* v, uint16_t* out,
                              int num_q, int num_kv, int hd, int seq_len) {
    const int gqa = num_q / num_kv, bpk = hd / OR_TQ_BLOCK;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int kvh = 0; kvh < num_kv; kvh++) {
        for (int db = 0; db < bpk; db++) {
            float acc[8][OR_TQ_BLOCK];
            memset(acc, 0, sizeof(acc));
            float x[OR_TQ_BLOCK];
            for (int pos = 0; pos < seq_len; pos++) {
                legacy_tq3_block_f32(v + ((int64_t)pos * num_kv + kvh) * bpk + db, x);
                for (int qi = 0; qi < gqa && qi < 8; qi++) {
                    const float p = probs[(int64_t)(kvh * gqa + qi) * seq_len + pos];
                    for (int l = 0; l < OR_TQ_BLOCK; l++) acc[qi][l] = fmaf(p, x[l], acc[qi][l]);
                }
            }
            for (int qi = 0; qi < gqa && qi < 8; qi++)
                for (int l = 0; l < OR_TQ_BLOCK; l++)
                    out[(int64_t)(kvh * gqa + qi) * hd + db * OR_TQ_BLOCK + l] = or_f32_to_f16(acc[qi][l]);
        }
    }
}

/* The fp16 scratch a legacy consumer reads: dequantized rows (TQ3 bulk
 * dequantization turboquant.cuh:169-200, Q8 attention.cuh:2614-2626) or the
 * fp16 cache itself. */
static uint16_t* legacy_scratch(int kind, const void* cache, int num_kv, int hd, int seq_len) {
    uint16_t* s = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)seq_len * num_kv * hd);
    #pragma omp parallel for schedule(static)
    for (int pos = 0; pos < seq_len; pos++)
        for (int h = 0; h < num_kv; h++)
            decode_row(kind, cache, pos, num_kv, h, hd, s + ((int64_t)pos * num_kv + h) * hd);
    return s;
}

int or_legacy_decode(int k_kind, int v_kind, int tq_fused, const uint16_t* q, const void* k,
                     const void* v, uint16_t* out, float* probs, int num_q, int num_kv, int hd,
                     int seq_len, float scale) {
    if (seq_len < 1 || hd % 32 || hd > 512 || num_q % num_kv || num_q / num_kv > 8) return -1;
    if (tq_fused && (k_kind == OR_KV_TQ3 || v_kind == OR_KV_TQ3) && hd % OR_TQ_BLOCK) return -1;
    float* sc = probs ? probs : (float*)malloc(sizeof(float) * (size_t)num_q * seq_len);
    if (k_kind == OR_KV_TQ3 && tq_fused) {
        legacy_scores_tq3(q, (const or_block_tq3*)k, sc, num_q, num_kv, hd, seq_len, scale);
    } else {
        uint16_t* k16 = legacy_scratch(k_kind, k, num_kv, hd, seq_len);
        legacy_scores_h(q, k16, sc, num_q, num_kv, hd, seq_len, scale);
        free(k16);
    }
    legacy_softmax(sc, num_q, seq_len);
    if (v_kind == OR_KV_TQ3 && tq_fused) {
        legacy_values_tq3(sc, (const or_block_tq3*)v, out, num_q, num_kv, hd, seq_len);
    } else {
        uint16_t* v16 = legacy_scratch(v_kind, v, num_kv, hd, seq_len);
        legacy_values_h(sc, v16, out, num_q, num_kv, hd, seq_len);
        free(v16);
    }
    if (!probs) free(sc);
    return 0;
}

/* ===================================================================== */
/* DFK2 KV-inject planes                                                  */
/* ===================================================================== */
/* dfki2_dequant_kernel (model.cuh:149-159): out[i] = half(float(q[i]) *
 * float(s[row * (kv_dim / 128) + col / 128])), row = i / kv_dim. */
void or_dfk2_dequant(const int8_t* q, const uint16_t* s, uint16_t* out, int64_t n, int kv_dim) {
    for (int64_t i = 0; i < n; i++) {
        const int col = (int)(i % kv_dim);
        const int64_t row = i / kv_dim;
        const float sc = or_f16_to_f32(s[row * (kv_dim / 128) + col / 128]);
        out[i] = or_f32_to_f16((float)q[i] * sc);
    }
}

/* ===================================================================== */
/* Block-sparse TQ3 verify (attention.cuh:2193-2533; sparse_index.cuh:214) */
/* ===================================================================== */

/* tq3_kpool_ms_update_kern (attention.cuh:2445-2533): for position blocks
 * n = blk_lo .. ceil(total_kv / bsn) - 1 of each kv head, the fp16 mean and
 * sign-preserving max-abs over the block's dequantized fp16 K rows (the same
 * values as the bulk dequantization): sum += x in position order, mean =
 * sum / n_pos; max-abs keeps the first largest |x|, starting from 0. */
void or_tq3_kpool_update(const or_block_tq3* k, uint16_t* k_pool, uint16_t* k_pool_max,
                         int num_kv, int hd, int total_kv, int blk_lo, int n_blocks_stride,
                         int bsn) {
    const int cur_blocks = (total_kv + bsn - 1) / bsn;
    const int bpk = hd / OR_TQ_BLOCK;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < num_kv; h++) {
        for (int n = blk_lo; n < cur_blocks; n++) {
            const int t_lo = n * bsn;
            const int t_hi = t_lo + bsn < total_kv ? t_lo + bsn : total_kv;
            const int64_t ob = ((int64_t)h * n_blocks_stride + n) * hd;
            if (t_lo >= t_hi) {
                for (int c = 0; c < hd; c++) k_pool[ob + c] = k_pool_max[ob + c] = 0;
                continue;
            }
            const int n_pos = t_hi - t_lo;
            uint16_t* rows = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n_pos * hd);
            for (int pp = 0; pp < n_pos; pp++)
                for (int j = 0; j < bpk; j++)
                    tq3_decode_one(k + ((int64_t)(t_lo + pp) * num_kv + h) * bpk + j,
                                   rows + (int64_t)pp * hd + j * OR_TQ_BLOCK, NULL);
            for (int c = 0; c < hd; c++) {
                float sum = 0.0f, best_mag = 0.0f, best_val = 0.0f;
                for (int pp = 0; pp < n_pos; pp++) {
                    const float x = or_f16_to_f32(rows[(int64_t)pp * hd + c]);
                    sum += x;
                    const float mg = fabsf(x);
                    if (mg > best_mag) { best_mag = mg; best_val = x; }
                }
                k_pool[ob + c] = or_f32_to_f16(sum / (float)n_pos);
                k_pool_max[ob + c] = or_f32_to_f16(best_val);
            }
            free(rows);
        }
    }
}

/* build_block_index_ms_kern (sparse_attn/sparse_index.cuh:214-330) for one
 * (kv_head, t_idx): q_avg = fp16(sum over the GQA heads * (1/GQA)); block
 * score max(q_avg . mean, beta * q_avg . maxabs) over half2 pairs (each pair
 * sum rounded once, products exact), -inf past the causal block
 * (start_pos + t_idx) / bsn; top_k picks of the highest score, the lower
 * block index on ties, never a -inf (or NaN) score; the picks sorted
 * ascending, then -1 padding. */
/* The block scores of one (kv_head, t_idx) into sc[n_blocks] (the first
 * half of build_block_index_ms_kern, sparse_index.cuh:243-290). */
static void block_scores_one(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                             float* sc, int h, int t, int num_q, int num_kv, int hd, int start_pos,
                             int bsn, int n_blocks, int n_blocks_stride, float beta) {
    const int gqa = num_q / num_kv;
    const float inv_g = 1.0f / (float)gqa;
    float* qa = (float*)malloc(sizeof(float) * hd);
    for (int c = 0; c < hd; c++) {
        float s = 0.0f;
        for (int g = 0; g < gqa; g++)
            s += or_f16_to_f32(q[((int64_t)t * num_q + h * gqa + g) * hd + c]);
        qa[c] = or_f16_to_f32(or_f32_to_f16(s * inv_g));
    }
    const int causal_max = (start_pos + t) / bsn;
    for (int n = 0; n < n_blocks; n++) {
        const uint16_t* mn = k_pool + ((int64_t)h * n_blocks_stride + n) * hd;
        const uint16_t* mx = k_pool_max + ((int64_t)h * n_blocks_stride + n) * hd;
        float s_mean = 0.0f, s_max = 0.0f;
        for (int c = 0; c < hd; c += 2) {
            s_mean += qa[c] * or_f16_to_f32(mn[c]) + qa[c + 1] * or_f16_to_f32(mn[c + 1]);
            s_max += qa[c] * or_f16_to_f32(mx[c]) + qa[c + 1] * or_f16_to_f32(mx[c + 1]);
        }
        float s = fmaxf(s_mean, beta * s_max);
        if (n > causal_max) s = -INFINITY;
        sc[n] = s;
    }
    free(qa);
}

/* Block scores [num_kv][sub_n][n_blocks] as build_block_index_ms_kern forms them. */
void or_block_scores_ms(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                        float* scores, int num_q, int num_kv, int hd, int sub_n, int start_pos,
                        int bsn, int n_blocks, int n_blocks_stride, float beta) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < num_kv; h++)
        for (int t = 0; t < sub_n; t++)
            block_scores_one(q, k_pool, k_pool_max, scores + ((int64_t)h * sub_n + t) * n_blocks, h, t,
                             num_q, num_kv, hd, start_pos, bsn, n_blocks, n_blocks_stride, beta);
}

void or_block_index_ms(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                       int32_t* block_index, int num_q, int num_kv, int hd, int sub_n,
                       int sub_n_max, int start_pos, int top_k, int bsn, int n_blocks,
                       int n_blocks_stride, float beta) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < num_kv; h++) {
        for (int t = 0; t < sub_n; t++) {
            float* sc = (float*)malloc(sizeof(float) * (n_blocks > 0 ? n_blocks : 1));
            block_scores_one(q, k_pool, k_pool_max, sc, h, t, num_q, num_kv, hd, start_pos, bsn,
                             n_blocks, n_blocks_stride, beta);
            int32_t* row = block_index + ((int64_t)h * sub_n_max + t) * top_k;
            int k = 0;
            for (; k < top_k; k++) {
                float lb = -INFINITY;
                int li = -1;
                for (int n = 0; n < n_blocks; n++)
                    if (sc[n] > lb) { lb = sc[n]; li = n; }
                if (li < 0) break;
                row[k] = li;
                sc[li] = -INFINITY;
            }
            for (int kk = k; kk < top_k; kk++) row[kk] = -1;
            for (int i = 1; i < k; i++) {      /* ascending */
                const int32_t x = row[i];
                int j = i;
                while (j > 0 && row[j - 1] > x) { row[j] = row[j - 1]; j--; }
                row[j] = x;
            }
            free(sc);
        }
    }
}

/* flash_attn_chunk_block_sparse_split_tq3 (attention.cuh:2193-2433): split
 * z takes entries [z * per, min((z + 1) * per, top_k)) of the query's block
 * list (per = ceil(top_k / k_splits)), stops at a -1, and runs the dense
 * kernel's tile body over each block's BM = 32 tiles up to start_pos + t. */
void or_attn_block_sparse_split(const uint16_t* q, const or_block_tq3* k, const or_block_tq3* v,
                                const int32_t* block_index, float* part_m, float* part_l,
                                float* part_o, int num_q, int num_kv, int hd, int start_pos,
                                int sub_n, int sub_n_max, float scale, int top_k, int bsn,
                                int k_splits, const uint32_t* tree_mask) {
    const int gqa = num_q / num_kv;
    #pragma omp parallel for collapse(3) schedule(dynamic)
    for (int h = 0; h < num_kv; h++) {
        for (int t = 0; t < sub_n; t++) {
            for (int z = 0; z < k_splits; z++) {
                const int abs_pos = start_pos + t, active_end_t = abs_pos + 1;
                const int per = (top_k + k_splits - 1) / k_splits;
                const int tk_lo = z * per;
                const int tk_hi = (z + 1) * per < top_k ? (z + 1) * per : top_k;
                const int32_t* bi = block_index + ((int64_t)h * sub_n_max + t) * top_k;
                split_state st;
                split_state_init(&st, q, num_q, num_kv, hd, h, t);
                for (int tk = tk_lo; tk < tk_hi; tk++) {
                    const int blk = bi[tk];
                    if (blk < 0) break;
                    for (int inner = 0; inner < bsn / OR_BM; inner++) {
                        const int ts = blk * bsn + inner * OR_BM;
                        if (ts > abs_pos) break;
                        const int te = ts + OR_BM < active_end_t ? ts + OR_BM : active_end_t;
                        if (te - ts <= 0) continue;
                        split_tile(&st, OR_KV_TQ3, k, v, num_kv, hd, gqa, start_pos, scale,
                                   tree_mask, h, t, ts, te - ts);
                    }
                }
                split_state_store(&st, part_m, part_l, part_o, num_q, num_kv, hd, sub_n_max,
                                  k_splits, h, t, z);
            }
        }
    }
}
