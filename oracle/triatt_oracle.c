/*
 * CPU restatement of TriAttention's quantize-and-attend arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker.  The product path (triattention_amd) never calls it.
 *
 * Every function follows one reference routine (paths relative to the
 * reference repository root, triattention/kernels/...):
 *   ora_rotate128     cuda/prefill_sm80.cu:95-115       (rotate128, kRotationSigns)
 *   ora_quantize_q    cuda/common_device.cuh:1-28       (quantize_q_kernel)
 *   ora_stats         cuda/common_device.cuh:30-56      (partial_kernel, finalize_kernel)
 *   ora_quantize_k    cuda/common_device.cuh:58-131     (quantize_k_kernel)
 *   ora_pack_v        cuda/common_device.cuh:132-172    (vnorm, pack_v_kernel)
 *   ora_prefill       cuda/prefill_sm80.cu:244-488      (scaled_row_max, tile_base_margin, run_task)
 *   ora_decode        cuda/common_device.cuh:178-469    (decode_tile, decode_kernel, decode_merge_kernel)
 *                     kernels/decode.py:17-67           (tile states, kept-tile lists, V recency rule)
 *   grown_state/vfmt  extension, no reference counterpart: tiles taken from a full tail after the
 *                     prompt's (the reference overwrites the tail's last slot, common_device.cuh:384)
 *
 * Arithmetic conventions (the defined semantics that the HIP kernels match):
 *  - IEEE-754 binary32 with round-to-nearest-even and denormals kept.  The
 *    reference was built with --use_fast_math; its approximate division,
 *    reciprocal and exp2 are replaced by IEEE division and by ora_texp2 below.
 *  - ora_texp2 is the one exp2 of the oracle: x clamped to >= -125,
 *    n = rint(x), f = x - n, a degree-6 polynomial for 2^f evaluated by fmaf
 *    in Horner order, scaled by 2^n.  Max error 0.952 ulp over [-125, 0].
 *    The GPU kernels compute the same function for the per-tile factors and
 *    the merge weights (n from the 1.5*2^23 shifter, added to the exponent
 *    field; ora_texp2_shifter restates that form so tests can pin the
 *    equality).  For the per-score probabilities (P levels, fp16 P) they use
 *    the hardware exp2 (v_exp_f32, ~1 ulp), as the reference uses the
 *    hardware ex2.approx: a P level then differs from this oracle's only
 *    where e * levels falls within a few ulp of a rounding boundary, and
 *    the outputs stay far inside the parity tolerance.
 *  - Per-element expressions that decide discrete values (codes, P levels,
 *    fp16 probabilities) follow the reference's operation sequence literally,
 *    including the 1.5*2^23 "magic" offset in the 8-bit score argument
 *    (prefill_sm80.cu:317-320) and the 49152.5 magic of the P quantizer
 *    (prefill_sm80.cu:78, :398-403).
 *  - Accumulators are exact restatements: integer MMA results are exact
 *    integers and the magic-offset bookkeeping `corr` of the reference
 *    (prefill_sm80.cu:350-357, :448) is identically zero here.
 *
 * Build: see oracle/Makefile (gcc, -ffp-contract=off, OpenMP).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define D 128
#define BN 64
#define STAT_BLOCKS 64
#define MAGIC_F 12582912.0f /* 1.5 * 2^23, prefill_sm80.cu:27 */
#define PMAGIC_HALF 49152.5f /* prefill_sm80.cu:78 */
#define NEAR_V8 16           /* decode.py:9 */

static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bf16f(uint16_t h) { return bitsf((uint32_t)h << 16); }

/* ------------------------------------------------------------------ exp2 */
/* 2^f = 1 + f P(f) on [-0.5, 0.5]: P is the polynomial of exp2f in S. L. Moshier's Cephes Math
 * Library (single precision) with its coefficients rounded to binary32 (max error 0.952 ulp, exhaustive). */
static const float EXP2_C[7] = {
    0x1.000000p+0f, 0x1.62e430p-1f, 0x1.ebfbdcp-3f, 0x1.c6aee8p-5f,
    0x1.3b2d4cp-7f, 0x1.5f3e52p-10f, 0x1.41fbbcp-13f};

float ora_texp2(float x) {
  x = fmaxf(x, -125.0f);
  const float n = rintf(x);
  const float f = x - n;
  float p = EXP2_C[6];
  for (int k = 5; k >= 0; --k) p = fmaf(p, f, EXP2_C[k]);
  return ldexpf(p, (int)n);
}

void ora_texp2_batch(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = ora_texp2(x[i]);
}

/* The GPU kernels' form of texp2 (csrc/common.h): t = x + 1.5*2^23 rounds to
 * nearest even and holds n = rint(x) in its low mantissa bits; 2^n is applied
 * by adding (bits(t) << 23) to the bits of the polynomial. */
float ora_texp2_shifter(float x) {
  x = fmaxf(x, -125.0f);
  volatile float t = x + MAGIC_F;
  const float n = t - MAGIC_F;
  const float f = x - n;
  float p = EXP2_C[6];
  for (int k = 5; k >= 0; --k) p = fmaf(p, f, EXP2_C[k]);
  return bitsf(fbits(p) + (fbits(t) << 23));
}

void ora_texp2_shifter_batch(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = ora_texp2_shifter(x[i]);
}

/* ------------------------------------------------------- fp16 / bf16 RNE */
uint16_t ora_f32_to_f16(float f) {
  const uint32_t u = fbits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
  const int e = (int)(a >> 23) - 127;
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) { /* normal half */
    uint32_t m = a & 0x7fffffu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* may carry into exponent: correct */
    return (uint16_t)(sign | h);
  }
  /* subnormal half: value = q * 2^-24 */
  if (e < -25) return (uint16_t)sign;
  const uint32_t m = (a & 0x7fffffu) | 0x800000u; /* 24-bit significand, value = m * 2^(e-23) */
  const int shift = -e - 1;                       /* q = m >> (shift) with e-23+shift = -24 */
  uint32_t q = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

float ora_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
  return bitsf(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t ora_f32_to_bf16(float f) {
  const uint32_t u = fbits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

/* -------------------------------------------------------------- rotation */
static const uint32_t ROT_SIGNS[4] = {0x9a3b5e71u, 0x2c6d8f13u, 0xe41b7a95u, 0x5f02c3d8u};

/* y = c * H128 * (s .* x); butterflies over index bits 0..6 in that order,
 * each mapping (lo, hi) -> (lo + hi, lo - hi)  (prefill_sm80.cu:96-115). */
void ora_rotate128(float* x) {
  for (int c = 0; c < D; ++c)
    if ((ROT_SIGNS[c >> 5] >> (c & 31)) & 1u) x[c] = -x[c];
  for (int bit = 1; bit < D; bit <<= 1)
    for (int i = 0; i < D; ++i)
      if (!(i & bit)) {
        const float lo = x[i], hi = x[i | bit];
        x[i] = lo + hi;
        x[i | bit] = lo - hi;
      }
  for (int c = 0; c < D; ++c) x[c] *= 0.08838834764831845f;
}

/* ---------------------------------------------------------- Q quantizer */
/* One rotated row -> INT8 codes (and INT4 nibbles, low nibble = even feature).
 * common_device.cuh:1-28. */
static void quantize_row(const float* y, int8_t* q8, float* qa, uint8_t* q4, float* qa4) {
  float m = 0.f;
  for (int c = 0; c < D; ++c) m = fmaxf(m, fabsf(y[c]));
  const float inv = m > 0.f ? 127.f / m : 0.f;
  for (int c = 0; c < D; ++c) q8[c] = (int8_t)(int)rintf(y[c] * inv);
  *qa = m / 127.f;
  if (q4) {
    const float inv4 = m > 0.f ? 7.f / m : 0.f;
    for (int c = 0; c < D; c += 2) {
      const int lo = (int)rintf(y[c] * inv4), hi = (int)rintf(y[c + 1] * inv4);
      q4[c / 2] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
    }
    *qa4 = m / 7.f;
  }
}

void ora_quantize_q(const uint16_t* q, int64_t sh, int64_t st, int hq, int t, int8_t* q8, float* qa,
                    uint8_t* q4, float* qa4) {
  for (int h = 0; h < hq; ++h)
    for (int r = 0; r < t; ++r) {
      float y[D];
      for (int c = 0; c < D; ++c) y[c] = bf16f(q[h * sh + (int64_t)r * st + c]);
      ora_rotate128(y);
      const int64_t row = (int64_t)h * t + r;
      quantize_row(y, q8 + row * D, qa + row, q4 ? q4 + row * (D / 2) : NULL, q4 ? qa4 + row : NULL);
    }
}

/* --------------------------------------------------------------- stats */
/* partial [h][64][3][128] = per block b: sequential sum, max, min over tokens
 * t = b, b+64, ...; stat [h][3][128] = mean, scale, 1/scale with the blocks
 * summed in block order (common_device.cuh:32-56). */
void ora_stats(const uint16_t* x, int64_t sh, int64_t st, int h, int t, int identity, float* partial,
               float* stat) {
  for (int hd = 0; hd < h; ++hd)
    for (int c = 0; c < D; ++c) {
      float sum2 = 0.f, hi2 = -FLT_MAX, lo2 = FLT_MAX;
      for (int b = 0; b < STAT_BLOCKS; ++b) {
        float sum = 0.f, hi = -FLT_MAX, lo = FLT_MAX;
        for (int tk = b; tk < t; tk += STAT_BLOCKS) {
          const float v = bf16f(x[hd * sh + (int64_t)tk * st + c]);
          sum += v;
          hi = fmaxf(hi, v);
          lo = fminf(lo, v);
        }
        if (partial) {
          float* o = partial + (((int64_t)hd * STAT_BLOCKS + b) * 3) * D + c;
          o[0] = sum; o[D] = hi; o[2 * D] = lo;
        }
        sum2 += sum;
        hi2 = fmaxf(hi2, hi);
        lo2 = fminf(lo2, lo);
      }
      float mean = 0.f, scale = 1.f;
      if (!identity) {
        mean = sum2 / (float)t;
        const float range = fmaxf(hi2 - mean, mean - lo2);
        scale = range > 0.f ? range / 127.f : 1.f;
      }
      stat[(int64_t)hd * 3 * D + c] = mean;
      stat[(int64_t)hd * 3 * D + D + c] = scale;
      stat[(int64_t)hd * 3 * D + 2 * D + c] = 1.f / scale;
    }
}

/* ----------------------------------------------------------- K quantizer */
/* Logical outputs: k8/k4 [hk][tiles*64][128] signed codes, ka/ka4 [hk][tiles][4].
 * y = R(k - mean) per key (zero for padded keys); per 16-key group absmax
 * scale (common_device.cuh:58-131). */
void ora_quantize_k(const uint16_t* k, int64_t sh, int64_t st, int hk, int t, const float* kstat, int8_t* k8,
                    float* ka, int8_t* k4, float* ka4) {
  const int tiles = (t + BN - 1) / BN;
  float* y = (float*)malloc(sizeof(float) * BN * D);
  for (int h = 0; h < hk; ++h) {
    const float* mean = kstat + (int64_t)h * 3 * D;
    for (int tile = 0; tile < tiles; ++tile) {
      for (int r = 0; r < BN; ++r) {
        const int tk = tile * BN + r;
        for (int c = 0; c < D; ++c) y[r * D + c] = tk < t ? bf16f(k[h * sh + (int64_t)tk * st + c]) - mean[c] : 0.f;
        ora_rotate128(y + r * D);
      }
      for (int g = 0; g < 4; ++g) {
        float cm = 0.f;
        for (int i = 0; i < 16 * D; ++i) cm = fmaxf(cm, fabsf(y[g * 16 * D + i]));
        const float inv = cm > 0.f ? 127.f / cm : 0.f, inv4 = cm > 0.f ? 7.f / cm : 0.f;
        const int64_t si = ((int64_t)h * tiles + tile) * 4 + g;
        ka[si] = cm > 0.f ? cm / 127.f : 1.f;
        if (k4) ka4[si] = cm > 0.f ? cm / 7.f : 1.f;
        for (int r = g * 16; r < g * 16 + 16; ++r) {
          const int64_t row = ((int64_t)h * tiles + tile) * BN + r;
          for (int c = 0; c < D; ++c) {
            k8[row * D + c] = (int8_t)(int)rintf(y[r * D + c] * inv);
            if (k4) {
              const int v = (int)rintf(y[r * D + c] * inv4);
              k4[row * D + c] = (int8_t)(((v & 15) ^ 8) - 8); /* the 4-bit field, sign-extended */
            }
          }
        }
      }
    }
  }
  free(y);
}

/* ------------------------------------------------------------- V packer */
/* Logical outputs [hk][tiles*64][128]: v16 fp16 bits of v', v8 = clamp(rint(v'),
 * +-127), v4 = clamp(rint(v' * f32(7/127)), +-7) with v' = (v - mean) * inv,
 * zero for padded keys (common_device.cuh:132-172). */
void ora_pack_v(const uint16_t* v, int64_t sh, int64_t st, int hk, int t, const float* vstat, uint16_t* v16,
                int8_t* v8, int8_t* v4) {
  const int tiles = (t + BN - 1) / BN;
  for (int h = 0; h < hk; ++h) {
    const float* mean = vstat + (int64_t)h * 3 * D;
    const float* inv = mean + 2 * D;
    for (int tk = 0; tk < tiles * BN; ++tk)
      for (int c = 0; c < D; ++c) {
        const float vn = tk < t ? (bf16f(v[h * sh + (int64_t)tk * st + c]) - mean[c]) * inv[c] : 0.f;
        const int64_t i = ((int64_t)h * tiles * BN + tk) * D + c;
        if (v16) v16[i] = ora_f32_to_f16(vn);
        if (v8) {
          int q = (int)rintf(vn);
          v8[i] = (int8_t)(q < -127 ? -127 : q > 127 ? 127 : q);
        }
        if (v4) {
          int q = (int)rintf(vn * (7.f / 127.f));
          v4[i] = (int8_t)(q < -7 ? -7 : q > 7 ? 7 : q);
        }
      }
  }
}

/* ---------------------------------------------------- band classification */
/* Tile lists of one (q-head band, query tile qb): prefill_sm80.cu:280-286. */
typedef struct { int n16, lo8, n8, lo4, n4; } lists_t;

static lists_t band_lists(int w8, int w4, int qb) {
  lists_t l;
  l.n16 = qb > 0 ? 2 : 1;
  l.lo8 = qb - w8 + 1 > 1 ? qb - w8 + 1 : 1;
  l.n8 = qb - l.lo8 > 0 ? qb - l.lo8 : 0;
  l.lo4 = qb - w4 + 1 > 1 ? qb - w4 + 1 : 1;
  l.n4 = qb - w8 - l.lo4 + 1 > 0 ? qb - w8 - l.lo4 + 1 : 0;
  return l;
}

/* Visit-order tile list and pass kind of every entry; returns the count.
 * kind: 0 = F16 (INT8 QK, fp16 PV), 1 = I8 (INT8 QK, u8 x s8 PV),
 *       2 = Q4 (INT4 QK, u8 x s8 PV). */
int ora_band_tiles(int w8, int w4, int qb, int* cols, int* kind) {
  const lists_t l = band_lists(w8, w4, qb);
  int n = 0;
  cols[n] = 0; kind[n++] = 0;
  if (qb > 0) { cols[n] = qb; kind[n++] = 0; }
  for (int i = 0; i < l.n8; ++i) { cols[n] = l.lo8 + i; kind[n++] = 1; }
  for (int i = 0; i < l.n4; ++i) { cols[n] = l.lo4 + i; kind[n++] = 2; }
  return n;
}

/* Planted mistakes for the tests of the oracle's own pins (never set outside those tests): each
 * value replaces one step of the quantized-P rules by a plausible wrong form, so that a test can show
 * that its independent check detects it.  0 = the reference's rules. */
enum {
  MUT_NONE = 0,
  MUT_NO_MARGIN = 1,     /* base = tile max, no margin */
  MUT_NO_HALF = 2,       /* prefill P levels: floor(x) instead of floor(x + 0.5) */
  MUT_DITHER_BYTE = 3,   /* decode dither from bits 8-15 of the dot product, not bits 0-7 */
  MUT_NO_REL_MARGIN = 4, /* margin without its |base| * 2.4e-7 term */
  MUT_BQ_LEVELS = 5,     /* bq = 2^(base - m) / 256 instead of / levels */
  MUT_V4_RESTORE = 6,    /* INT4-V tiles weighted by bq, without the 127/7 restore */
  MUT_NO_DITHER = 7,     /* decode P levels without the dither (plain truncation) */
  MUT_SLOPE_GROUP = 8,   /* P-level arguments all use the first 16-key group's slope */
  MUT_GROWN_MASK = 9,    /* tiles taken from the tail masked like prompt tiles (keys past the prompt invalid) */
  MUT_GROWN_STATE = 10,  /* tiles taken from the tail classified against the prompt's tile count */
  MUT_EXP_UP = 11,       /* prefill per-score exp2 two ulps up (a hardware exp2 on the other side) */
  MUT_EXP_DOWN = 12,     /* the same, two ulps down */
};
static int g_mutation = MUT_NONE;
void ora_set_mutation(int m) { g_mutation = m; }

static inline float tile_base_margin(float slope, float base) {
  if (g_mutation == MUT_NO_MARGIN) return 0.f;
  if (g_mutation == MUT_NO_REL_MARGIN) return slope * 0.75f;
  return fmaf(slope, 0.75f, fabsf(base) * 2.4e-7f);
}

/* P level of one key: byte 1 of fma(e, levels, dither) (prefill_sm80.cu:398-403,
 * common_device.cuh:243-244). */
static inline int p_level(float e, float levels, float dither) { return (int)((fbits(fmaf(e, levels, dither)) >> 8) & 0xffu); }

static inline float pmagic_half(void) { return g_mutation == MUT_NO_HALF ? 49152.0f : PMAGIC_HALF; }
static inline float level_scale(float levels) { return g_mutation == MUT_BQ_LEVELS ? 256.f : levels; }

/* Per-tile record of one query row (prefill) or one q-head (decode), for the tests that check the
 * oracle's quantized-P rules tile by tile against an independent float64 evaluation. */
typedef struct {
  int cap, n;
  int32_t *col, *kind, *split;
  float *m, *base, *bq;
  int32_t* p; /* [cap][64]: P levels (quantized tiles) or the fp16 bits of p (F16 tiles) */
} ora_trace;

static void trace_tile(ora_trace* tr, int col, int kind, int split, float m, float base, float bq, const int* p) {
  if (!tr || tr->n >= tr->cap) return;
  const int e = tr->n++;
  tr->col[e] = col;
  tr->kind[e] = kind;
  if (tr->split) tr->split[e] = split;
  tr->m[e] = m;
  tr->base[e] = base;
  tr->bq[e] = bq;
  for (int k = 0; k < BN; ++k) tr->p[(int64_t)e * BN + k] = p[k];
}

/* ------------------------------------------------------------- prefill */
/* One query row of run_task (prefill_sm80.cu:259-488), exact-accumulator form.
 * Codes are logical: q8 [hq][t][128], q4 packed [hq][t][64] (low nibble = even
 * feature), k8/k4 [hk][tiles*64][128] signed, v16 fp16 bits, v8 signed. */
typedef struct {
  int hq, hk, t;
  const int32_t* bands;
  float sm_log2;
  const int8_t *q8, *k8, *k4, *v8;
  const uint8_t* q4;
  const float *qa, *ka, *qa4, *ka4, *vstat;
  const uint16_t* v16;
} prefill_args;

/* exp2 results two ulps either side of e: the hardware exp2 of the kernels' per-score probabilities
 * (v_exp_f32, within 1 ulp, like the reference's ex2.approx) and texp2 (0.952 ulp) may differ by that. */
static void exp2_neighbours(float e, float* lo, float* hi) {
  *lo = nextafterf(nextafterf(e, -INFINITY), -INFINITY);
  *hi = nextafterf(nextafterf(e, INFINITY), INFINITY);
  if (*lo < 0.f) *lo = 0.f;
}

/* The per-score exp2 of prefill: texp2, or under MUT_EXP_UP / MUT_EXP_DOWN its neighbour two ulps away. */
static float score_exp2(float arg) {
  const float e = ora_texp2(arg);
  if (g_mutation != MUT_EXP_UP && g_mutation != MUT_EXP_DOWN) return e;
  float lo, hi;
  exp2_neighbours(e, &lo, &hi);
  return g_mutation == MUT_EXP_UP ? hi : lo;
}

/* tol_row (may be NULL): per channel, how far the output can move when every probability that a
 * two-ulp change of its exp2 would round to the next P level (quantized tiles) or fp16 value (F16
 * tiles) takes that neighbour: the sum of those steps times |V'|, through the denominator as well,
 * in output units.  Everywhere else the output is determined by the reference's operation sequence. */
static void prefill_row(const prefill_args* a, int qh, int i, float* out_row, ora_trace* tr, float* tol_row) {
  const int g = a->hq / a->hk, kh = qh / g, tiles = (a->t + BN - 1) / BN, qb = i / BN;
  const int64_t qrow = (int64_t)qh * a->t + i;
  int cols[4096], kind[4096];
  const int n = ora_band_tiles(a->bands[2 * qh], a->bands[2 * qh + 1], qb, cols, kind);
  int8_t q4c[D];
  if (a->q4)
    for (int c = 0; c < D; c += 2) {
      const uint8_t b = a->q4[qrow * (D / 2) + c / 2];
      q4c[c] = (int8_t)(((b & 15) ^ 8) - 8);
      q4c[c + 1] = (int8_t)(((b >> 4) ^ 8) - 8);
    }
  const float qs8 = a->qa[qrow] * a->sm_log2;
  const float qs4 = a->q4 ? a->qa4[qrow] * a->sm_log2 : 0.f;
  float m = -FLT_MAX, denom = 0.f;
  double acc64[D];
  float out[D];
  double amb[D], amb_den = 0.0;  /* ambiguity bound of out and denom (tol_row) */
  for (int c = 0; c < D; ++c) out[c] = 0.f, amb[c] = 0.0;
  int dot[BN], valid[BN];
  for (int e = 0; e < n; ++e) {
    const int col = cols[e], kd = kind[e];
    const int four = kd == 2;
    /* masking: only the last entry of a pass, when it is the query tile itself */
    const int last_of_pass = (e == n - 1) || (kind[e + 1] != kd);
    const int masked = last_of_pass && col == qb;
    const int8_t* qc = four ? q4c : a->q8 + qrow * D;
    const int8_t* kc = (four ? a->k4 : a->k8) + ((int64_t)kh * tiles + col) * BN * D;
    const float* ks = (four ? a->ka4 : a->ka) + ((int64_t)kh * tiles + col) * 4;
    const float qs = four ? qs4 : qs8;
    for (int k = 0; k < BN; ++k) {
      const int key = col * BN + k;
      valid[k] = !(masked && (key >= a->t || key > i));
      int s = 0;
      for (int c = 0; c < D; ++c) s += (int)qc[c] * (int)kc[(int64_t)k * D + c];
      dot[k] = s;
    }
    /* scaled_row_max (prefill_sm80.cu:244-253): per 16-key column the max raw
     * dot, scaled by RN(qs*ks[col]) */
    float tile = -INFINITY;
    float slope[4];
    for (int gc = 0; gc < 4; ++gc) {
      slope[gc] = qs * ks[gc];
      int have = 0, mx = 0;
      for (int k = gc * 16; k < gc * 16 + 16; ++k)
        if (valid[k] && (!have || dot[k] > mx)) { mx = dot[k]; have = 1; }
      if (have) tile = fmaxf(tile, slope[gc] * (float)mx);
    }
    const float nmax = fmaxf(m, tile);
    const float alpha = ora_texp2(m - nmax);
    m = nmax;
    for (int c = 0; c < D; ++c) out[c] = out[c] * alpha;
    if (tol_row) {
      for (int c = 0; c < D; ++c) amb[c] *= alpha;
      amb_den *= alpha;
    }
    if (kd == 0) {
      /* fp16 P x fp16 V' (prefill_sm80.cu:358-383) */
      denom *= alpha;
      uint16_t p16[BN];
      float pf[BN];
      for (int k = 0; k < BN; ++k) {
        const float x = valid[k] ? (float)dot[k] + MAGIC_F : -INFINITY;
        const float arg = fmaf(slope[k / 16], x, fmaf(-slope[k / 16], MAGIC_F, -m));
        const float e = score_exp2(arg);
        p16[k] = ora_f32_to_f16(e);
        pf[k] = ora_f16_to_f32(p16[k]);
        if (tol_row) {
          float lo, hi;
          exp2_neighbours(e, &lo, &hi);
          const double step = fmax(fabs((double)ora_f16_to_f32(ora_f32_to_f16(lo)) - pf[k]),
                                   fabs((double)ora_f16_to_f32(ora_f32_to_f16(hi)) - pf[k]));
          if (step > 0.0) {
            const uint16_t* vr = a->v16 + (((int64_t)kh * tiles + col) * BN + k) * D;
            amb_den += step;
            for (int c = 0; c < D; ++c) amb[c] += step * fabs((double)ora_f16_to_f32(vr[c]));
          }
        }
      }
      if (tr) {
        int pb[BN];
        for (int k = 0; k < BN; ++k) pb[k] = p16[k];
        trace_tile(tr, col, 0, 0, m, 0.f, 0.f, pb);
      }
      for (int kc16 = 0; kc16 < 4; ++kc16) {
        double s = 0.0;
        for (int k = kc16 * 16; k < kc16 * 16 + 16; ++k) s += (double)pf[k];
        denom = denom + (float)s;
      }
      const uint16_t* vt = a->v16 + ((int64_t)kh * tiles + col) * BN * D;
      for (int c = 0; c < D; ++c) acc64[c] = 0.0;
      for (int k = 0; k < BN; ++k) {
        if (pf[k] == 0.f) continue;
        for (int c = 0; c < D; ++c) acc64[c] += (double)pf[k] * (double)ora_f16_to_f32(vt[(int64_t)k * D + c]);
      }
      for (int c = 0; c < D; ++c) out[c] = (float)((double)out[c] + acc64[c]);
    } else {
      /* quantized P (u8) x INT8 V' (prefill_sm80.cu:384-449) */
      float ksmax = fmaxf(fmaxf(ks[0], ks[1]), fmaxf(ks[2], ks[3]));
      float base = tile > -INFINITY ? tile : m;
      base += tile_base_margin(qs * ksmax, base);
      const float bq = ora_texp2(base - m) / level_scale(255.f);
      int P[BN];
      int rs = 0;
      for (int k = 0; k < BN; ++k) {
        const float x = valid[k] ? (float)dot[k] : -INFINITY;
        const float sl = g_mutation == MUT_SLOPE_GROUP ? slope[0] : slope[k / 16];
        float arg;
        if (four) arg = fmaf(sl, x, -base);
        else arg = fmaf(sl, x + MAGIC_F, fmaf(-sl, MAGIC_F, -base));
        const float e = score_exp2(arg);
        P[k] = p_level(e, 255.f, pmagic_half());
        rs += P[k];
        if (tol_row) {
          float lo, hi;
          exp2_neighbours(e, &lo, &hi);
          if (p_level(lo, 255.f, pmagic_half()) != P[k] || p_level(hi, 255.f, pmagic_half()) != P[k]) {
            const int8_t* vr = a->v8 + (((int64_t)kh * tiles + col) * BN + k) * D;
            amb_den += bq;
            for (int c = 0; c < D; ++c) amb[c] += (double)bq * abs((int)vr[c]);
          }
        }
      }
      trace_tile(tr, col, kd, 0, m, base, bq, P);
      denom = fmaf((float)rs, bq, denom * alpha);
      const int8_t* vt = a->v8 + ((int64_t)kh * tiles + col) * BN * D;
      int32_t pv[D];
      for (int c = 0; c < D; ++c) pv[c] = 0;
      for (int k = 0; k < BN; ++k) {
        if (!P[k]) continue;
        for (int c = 0; c < D; ++c) pv[c] += P[k] * (int)vt[(int64_t)k * D + c];
      }
      for (int c = 0; c < D; ++c) out[c] = fmaf((float)pv[c], bq, out[c]);
    }
  }
  const float inv = denom > 0.f ? 1.f / denom : 0.f;
  const float* mean = a->vstat + (int64_t)kh * 3 * D;
  const float* scale = mean + D;
  for (int c = 0; c < D; ++c) out_row[c] = fmaf(out[c] * inv, scale[c], mean[c]);
  if (tol_row) {
    /* |d(o / l)| <= (|do| + |o / l| |dl|) / (l - |dl|), with 1% on top for the fp32 roundings */
    const double den = (double)denom - amb_den;
    for (int c = 0; c < D; ++c) {
      const double o = (double)out[c] / (denom > 0.f ? (double)denom : 1.0);
      tol_row[c] = amb_den == 0.0 ? 0.f
                   : den > 0.0 ? (float)(1.01 * (amb[c] + fabs(o) * amb_den) / den * scale[c])
                               : INFINITY;
    }
  }
}

void ora_prefill(int hq, int hk, int t, const int32_t* bands, float sm_log2, const int8_t* q8, const float* qa,
                 const uint8_t* q4, const float* qa4, const int8_t* k8, const float* ka, const int8_t* k4,
                 const float* ka4, const uint16_t* v16, const int8_t* v8, const float* vstat, float* out,
                 float* tol, int nthreads) {
  prefill_args a = {hq, hk, t, bands, sm_log2, q8, k8, k4, v8, q4, qa, ka, qa4, ka4, vstat, v16};
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
  for (int64_t r = 0; r < (int64_t)hq * t; ++r) {
    const int qh = (int)(r / t), i = (int)(r % t);
    prefill_row(&a, qh, i, out + r * D, NULL, tol ? tol + r * D : NULL);
  }
  (void)nthreads;
}

/* The rows rows[0..nrows) (flat index qh * t + i) of ora_prefill's output, into out [nrows][128]:
 * every row is computed on its own, so a sample of a long prompt costs only its rows. */
void ora_prefill_rows(int hq, int hk, int t, const int32_t* bands, float sm_log2, const int8_t* q8, const float* qa,
                      const uint8_t* q4, const float* qa4, const int8_t* k8, const float* ka, const int8_t* k4,
                      const float* ka4, const uint16_t* v16, const int8_t* v8, const float* vstat,
                      const int64_t* rows, int64_t nrows, float* out, float* tol, int nthreads) {
  prefill_args a = {hq, hk, t, bands, sm_log2, q8, k8, k4, v8, q4, qa, ka, qa4, ka4, vstat, v16};
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t r = 0; r < nrows; ++r)
    prefill_row(&a, (int)(rows[r] / t), (int)(rows[r] % t), out + r * D, NULL, tol ? tol + r * D : NULL);
  (void)nthreads;
}

/* One row of ora_prefill with its per-tile record (visit order): tile, kind (0 F16, 1 I8, 2 Q4),
 * running max after the tile, base and bq (quantized tiles), and per key the P level or the fp16
 * bits of p.  Returns the number of visited tiles (at most cap are recorded). */
int ora_prefill_trace(int hq, int hk, int t, const int32_t* bands, float sm_log2, const int8_t* q8, const float* qa,
                      const uint8_t* q4, const float* qa4, const int8_t* k8, const float* ka, const int8_t* k4,
                      const float* ka4, const uint16_t* v16, const int8_t* v8, const float* vstat, int qh, int i,
                      int cap, int32_t* col, int32_t* kind, float* m, float* base, float* bq, int32_t* p,
                      float* out_row) {
  prefill_args a = {hq, hk, t, bands, sm_log2, q8, k8, k4, v8, q4, qa, ka, qa4, ka4, vstat, v16};
  ora_trace tr = {cap, 0, col, kind, NULL, m, base, bq, p};
  prefill_row(&a, qh, i, out_row, &tr, NULL);
  return tr.n;
}

/* --------------------------------------------------------------- decode */
/* Per-tile decode state of one q-head (decode.py:27-30): 8, 4 or 0 (skipped). */
int ora_decode_state(int w8, int w4, int tiles, int j) {
  const int d = tiles - 1 - j;
  return (j == 0 || d < w8) ? 8 : (d < w4 ? 4 : 0);
}

/* V format of tile j (decode.py:17-22): 1 = INT8 V, 2 = INT4 V. */
int ora_decode_vfmt(int tiles, int j) { return (tiles - 1 - j < NEAR_V8 || j == 0) ? 1 : 2; }

/* Tail growth (extension, no reference counterpart): a tile j taken from the tail after the prompt's
 * `tiles` tiles is classified as the newest tile of a cache of j + 1 tiles when it enters, and keeps
 * that classification; the prompt's tiles keep theirs (the reference never reclassifies a stored
 * tile).  Every key of such a tile is valid. */
static int grown_state(int w8, int w4, int tiles, int j) {
  if (g_mutation == MUT_GROWN_STATE) return ora_decode_state(w8, w4, tiles, j);
  return j < tiles ? ora_decode_state(w8, w4, tiles, j) : ora_decode_state(w8, w4, j + 1, j);
}
static int grown_vfmt(int tiles, int j) { return j < tiles ? ora_decode_vfmt(tiles, j) : ora_decode_vfmt(j + 1, j); }

/* Exact restatement of the 32-lane butterfly sum used by decode_merge_kernel
 * (common_device.cuh:397-415): lane l holds an fma chain over channels 4l..4l+3. */
static float tail_score(const uint16_t* qv, const uint16_t* kv, const float* kmean, float sm_log2) {
  float part[32];
  for (int l = 0; l < 32; ++l) {
    float p = 0.f;
    for (int i = 0; i < 4; ++i) {
      const int c = l * 4 + i;
      p = fmaf(bf16f(qv[c]), bf16f(kv[c]) - kmean[c], p);
    }
    part[l] = p;
  }
  for (int o = 16; o; o >>= 1) {
    float nx[32];
    for (int l = 0; l < 32; ++l) nx[l] = part[l] + part[l ^ o];
    memcpy(part, nx, sizeof(part));
  }
  return part[0] * sm_log2;
}

typedef struct {
  int hq, hk, prompt, per, max_tail;
  int ctiles; /* tiles per KV head in the code arrays: the prompt's, then those taken from the tail */
  const int32_t* bounds; /* NULL: uniform split of `per`; else [hk][nsplit + 1] entry bounds */
  int nsplit;
  const int32_t* bands;
  float sm_log2;
  const uint16_t* q;
  const int8_t *k8, *k4, *v8, *v4;
  const float *ka, *ka4, *vstat, *kstat;
  const uint16_t *ktail, *vtail, *kcur, *vcur;
  int64_t step;
} decode_args;

/* One query head of decode_kernel + decode_merge_kernel. */
static void decode_head(const decode_args* a, int qh, float* out_row, ora_trace* tr, float* tpm, float* tpl,
                        float* tpo) {
  const int g = a->hq / a->hk, kh = qh / g, tiles = (a->prompt + BN - 1) / BN, ct = a->ctiles;
  /* kept-tile list of this KV head: ascending tiles whose group state > 0 */
  int* entry = (int*)malloc(sizeof(int) * (ct > 0 ? ct : 1));
  int* kprec = (int*)malloc(sizeof(int) * (ct > 0 ? ct : 1));
  int* own = (int*)malloc(sizeof(int) * (ct > 0 ? ct : 1));
  int count = 0;
  for (int j = 0; j < ct; ++j) {
    int kv = 0;
    for (int h = 0; h < g; ++h) {
      const int s = grown_state(a->bands[2 * (kh * g + h)], a->bands[2 * (kh * g + h) + 1], tiles, j);
      if (s > kv) kv = s;
    }
    if (kv > 0) {
      entry[count] = j;
      kprec[count] = kv;
      own[count] = grown_state(a->bands[2 * qh], a->bands[2 * qh + 1], tiles, j) > 0;
      ++count;
    }
  }
  /* splits use the maximum count over KV heads (decode.py:35-36; common_host.cuh:55) */
  int maxn = 1;
  for (int h2 = 0; h2 < a->hk; ++h2) {
    int c2 = 0;
    for (int j = 0; j < ct; ++j) {
      int kv = 0;
      for (int h = 0; h < g; ++h) {
        const int s = grown_state(a->bands[2 * (h2 * g + h)], a->bands[2 * (h2 * g + h) + 1], tiles, j);
        if (s > kv) kv = s;
      }
      c2 += kv > 0;
    }
    if (c2 > maxn) maxn = c2;
  }
  const int splits = a->bounds ? a->nsplit : (maxn + a->per - 1) / a->per > 1 ? (maxn + a->per - 1) / a->per : 1;

  /* in-kernel Q quantization (common_device.cuh:291-315) */
  float y[D];
  for (int c = 0; c < D; ++c) y[c] = bf16f(a->q[(int64_t)qh * D + c]);
  ora_rotate128(y);
  float mq = 0.f;
  for (int c = 0; c < D; ++c) mq = fmaxf(mq, fabsf(y[c]));
  int8_t q8[D], q4[D];
  const float inv = mq > 0.f ? 127.f / mq : 0.f, inv4 = mq > 0.f ? 7.f / mq : 0.f;
  for (int c = 0; c < D; ++c) {
    q8[c] = (int8_t)(int)rintf(y[c] * inv);
    const int v = (int)rintf(y[c] * inv4);
    q4[c] = (int8_t)(((v & 15) ^ 8) - 8);
  }
  const float qscale = mq > 0.f ? mq / 127.f * a->sm_log2 : FLT_MIN;
  const float qscale4 = mq > 0.f ? mq / 7.f * a->sm_log2 : FLT_MIN;

  float* pm = (float*)malloc(sizeof(float) * splits);
  float* pl = (float*)malloc(sizeof(float) * splits);
  float* po = (float*)malloc(sizeof(float) * splits * D);
  for (int s = 0; s < splits; ++s) {
    int first = s * a->per, last = count < first + a->per ? count : first + a->per;
    if (a->bounds) {
      /* the caller's partition, clamped as the kernel clamps it: into [0, count), at most 64 per split */
      const int32_t* bd = a->bounds + (int64_t)kh * (a->nsplit + 1) + s;
      first = bd[0] < 0 ? 0 : bd[0] > count ? count : bd[0];
      last = bd[1] < first ? first : bd[1];
      if (last > count) last = count;
      if (last > first + 64) last = first + 64;
    }
    float m = -FLT_MAX, dw[4] = {0.f, 0.f, 0.f, 0.f}, out[D];
    for (int c = 0; c < D; ++c) out[c] = 0.f;
    for (int e = first; e < last; ++e) {
      const int j = entry[e], four = kprec[e] == 4, fmt = grown_vfmt(tiles, j);
      const float* kt = (four ? a->ka4 : a->ka) + ((int64_t)kh * ct + j) * 4;
      const float qs = four ? qscale4 : qscale;
      const int8_t* qc = four ? q4 : q8;
      const int8_t* kc = (four ? a->k4 : a->k8) + ((int64_t)kh * ct + j) * BN * D;
      float slope[4];
      for (int w = 0; w < 4; ++w) slope[w] = qs * kt[w];
      const float slope1 = qs * fmaxf(fmaxf(kt[0], kt[1]), fmaxf(kt[2], kt[3]));
      int dot[BN], valid[BN];
      for (int k = 0; k < BN; ++k) {
        int sdot = 0;
        for (int c = 0; c < D; ++c) sdot += (int)qc[c] * (int)kc[(int64_t)k * D + c];
        dot[k] = sdot;
        valid[k] = own[e] && ((j >= tiles && g_mutation != MUT_GROWN_MASK) || j * BN + k < a->prompt);
      }
      float tile = -INFINITY;
      for (int w = 0; w < 4; ++w) {
        int have = 0, mx = 0;
        for (int k = w * 16; k < w * 16 + 16; ++k)
          if (valid[k] && (!have || dot[k] > mx)) { mx = dot[k]; have = 1; }
        if (have) tile = fmaxf(tile, slope[w] * (float)mx);
      }
      const float nmax = fmaxf(m, tile), alpha = ora_texp2(m - nmax);
      m = nmax;
      if (alpha != 1.f)
        for (int c = 0; c < D; ++c) out[c] *= alpha;
      const float levels = fmt == 1 ? 255.f : 15.f;
      const int any = tile > -INFINITY;
      float base = any ? tile : nmax;
      base += tile_base_margin(slope1, base);
      const float bq = any ? ora_texp2(base - nmax) / level_scale(levels) : 0.f;
      const float restore = (fmt == 1 || g_mutation == MUT_V4_RESTORE) ? bq : bq * (127.f / 7.f);
      int P[BN];
      for (int k = 0; k < BN; ++k) {
        const int w = g_mutation == MUT_SLOPE_GROUP ? 0 : k / 16;
        const float xm = valid[k] ? (float)dot[k] + MAGIC_F : -INFINITY;
        float dither = bitsf((fbits(xm) & 0xffu) | 0x47400000u);
        if (g_mutation == MUT_DITHER_BYTE) dither = bitsf(((fbits(xm) >> 8) & 0xffu) | 0x47400000u);
        if (g_mutation == MUT_NO_DITHER) dither = 49152.0f;
        float arg;
        if (!four) {
          const float bias = -slope[w] * MAGIC_F;
          arg = fmaf(slope[w], xm, bias - base);
        } else {
          arg = fmaf(slope[w], xm - MAGIC_F, -base);
        }
        P[k] = p_level(ora_texp2(arg), levels, dither);
      }
      trace_tile(tr, j, kprec[e] | fmt << 4, s, m, base, bq, P);
      /* denominators per 16-key group, as 4 lanes x 4 keys with a butterfly
       * (common_device.cuh:246-251) */
      for (int w = 0; w < 4; ++w) {
        float part[4];
        for (int sub = 0; sub < 4; ++sub) {
          const int kb = w * 16;
          const int s4 = P[kb + sub * 2] + P[kb + sub * 2 + 1] + P[kb + 8 + sub * 2] + P[kb + 9 + sub * 2];
          part[sub] = (float)s4 * bq;
        }
        const float tot = (part[0] + part[1]) + (part[2] + part[3]);
        dw[w] = fmaf(dw[w], alpha, tot);
      }
      const int8_t* vt = (fmt == 1 ? a->v8 : a->v4) + ((int64_t)kh * ct + j) * BN * D;
      int32_t pv[D];
      for (int c = 0; c < D; ++c) pv[c] = 0;
      for (int k = 0; k < BN; ++k) {
        if (!P[k]) continue;
        for (int c = 0; c < D; ++c) pv[c] += P[k] * (int)vt[(int64_t)k * D + c];
      }
      for (int c = 0; c < D; ++c) out[c] = fmaf((float)pv[c], restore, out[c]);
    }
    pm[s] = m;
    pl[s] = dw[0] + dw[1] + dw[2] + dw[3];
    for (int c = 0; c < D; ++c) po[(int64_t)s * D + c] = out[c];
  }
  if (tpm) {
    memcpy(tpm, pm, sizeof(float) * splits);
    memcpy(tpl, pl, sizeof(float) * splits);
    memcpy(tpo, po, sizeof(float) * splits * D);
  }

  /* merge (common_device.cuh:373-469) */
  const int prior = (int)(a->step < a->max_tail - 1 ? a->step : a->max_tail - 1), tail = prior + 1;
  const float* kmean = a->kstat + (int64_t)kh * 3 * D;
  float* ts = (float*)malloc(sizeof(float) * tail);
  for (int t = 0; t < tail; ++t) {
    const uint16_t* kv = t < prior ? a->ktail + ((int64_t)kh * a->max_tail + t) * D : a->kcur + (int64_t)kh * D;
    ts[t] = tail_score(a->q + (int64_t)qh * D, kv, kmean, a->sm_log2);
  }
  float m = -FLT_MAX;
  for (int s = 0; s < splits; ++s) m = fmaxf(m, pm[s]);
  for (int t = 0; t < tail; ++t) m = fmaxf(m, ts[t]);
  float wl[4] = {0.f, 0.f, 0.f, 0.f}, wo[4][D];
  for (int w = 0; w < 4; ++w)
    for (int c = 0; c < D; ++c) wo[w][c] = 0.f;
  for (int w = 0; w < 4; ++w)
    for (int s = w; s < splits; s += 4) {
      const float wt = ora_texp2(pm[s] - m);
      wl[w] = fmaf(pl[s], wt, wl[w]);
      for (int c = 0; c < D; ++c) wo[w][c] = fmaf(po[(int64_t)s * D + c], wt, wo[w][c]);
    }
  const float* vmean = a->vstat + (int64_t)kh * 3 * D;
  const float* vscale = vmean + D;
  for (int c = 0; c < D; ++c) {
    float total = 0.f, acc = 0.f;
    for (int w = 0; w < 4; ++w) { total += wl[w]; acc += wo[w][c]; }
    acc = fmaf(acc, vscale[c], total * vmean[c]);
    for (int t = 0; t < prior; ++t) {
      const float e = ora_texp2(ts[t] - m);
      total += e;
      acc = fmaf(e, bf16f(a->vtail[((int64_t)kh * a->max_tail + t) * D + c]), acc);
    }
    const float e = ora_texp2(ts[prior] - m);
    total += e;
    acc = fmaf(e, bf16f(a->vcur[(int64_t)kh * D + c]), acc);
    out_row[c] = acc / total;
  }
  free(ts); free(pm); free(pl); free(po); free(entry); free(kprec); free(own);
}

void ora_decode(int hq, int hk, int prompt, const int32_t* bands, int per, float sm_log2, const uint16_t* q,
                const int8_t* k8, const float* ka, const int8_t* k4, const float* ka4, const int8_t* v8,
                const int8_t* v4, const float* vstat, const float* kstat, const uint16_t* ktail,
                const uint16_t* vtail, int max_tail, const uint16_t* kcur, const uint16_t* vcur, int64_t step,
                const int32_t* bounds, int nsplit, int ctiles, float* out) {
  decode_args a = {hq, hk, prompt, per < 1 ? 1 : per, max_tail, ctiles, bounds, nsplit < 1 ? 1 : nsplit, bands,
                   sm_log2, q, k8, k4, v8, v4, ka, ka4, vstat, kstat, ktail, vtail, kcur, vcur, step};
  for (int qh = 0; qh < hq; ++qh) decode_head(&a, qh, out + (int64_t)qh * D, NULL, NULL, NULL, NULL);
}

/* ora_decode for one q-head with its record: per kept tile (split order) the tile, kprec | fmt << 4,
 * split, running max after the tile, base, bq and the 64 P levels; the split partials pm / pl
 * [splits] and po [splits][128]; returns the number of tiles visited (at most cap recorded). */
int ora_decode_trace(int hq, int hk, int prompt, const int32_t* bands, int per, float sm_log2, const uint16_t* q,
                     const int8_t* k8, const float* ka, const int8_t* k4, const float* ka4, const int8_t* v8,
                     const int8_t* v4, const float* vstat, const float* kstat, const uint16_t* ktail,
                     const uint16_t* vtail, int max_tail, const uint16_t* kcur, const uint16_t* vcur, int64_t step,
                     const int32_t* bounds, int nsplit, int ctiles, int qh, int cap, int32_t* col, int32_t* kind,
                     int32_t* split, float* m, float* base, float* bq, int32_t* p, float* pm, float* pl, float* po,
                     float* out_row) {
  decode_args a = {hq, hk, prompt, per < 1 ? 1 : per, max_tail, ctiles, bounds, nsplit < 1 ? 1 : nsplit, bands,
                   sm_log2, q, k8, k4, v8, v4, ka, ka4, vstat, kstat, ktail, vtail, kcur, vcur, step};
  ora_trace tr = {cap, 0, col, kind, split, m, base, bq, p};
  decode_head(&a, qh, out_row, &tr, pm, pl, po);
  return tr.n;
}

int ora_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
