// Shared device helpers for the gfx950 TriAttention kernels.
//
// Record layouts (one record = one 64-key tile of one KV head).  Sizes match the
// reference's record word counts (triattention/kernels/decode.py:7-8,
// cuda/prefill_sm80.cu:17-22); the byte order inside a record is chosen so that
// each 1 KiB "fragment" is exactly one operand of a 32x32 MFMA, loaded with one
// 16-byte access per lane (4-bit records pair two fragments per 16 bytes):
//
//   K8  8192 B  fragment F = kb*4 + ks (kb: 32-key block, ks: 32-feature step)
//               lane L byte j  <->  key kb*32 + L%32, feature ks*32 + 16*(L/32) + j
//   K4  4096 B  the 4-bit codes of the K8 layout; fragment F's lane L word pair
//               (w0, w1) sits at byte (F/2)*1024 + 16*L + 8*(F%2), so one 16-byte
//               access per lane fetches fragments 2P and 2P+1.  K8-layout byte j is
//               the low nibble of w0 byte j (j<4), high nibble of w0 byte j-4 (j<8),
//               low nibble of w1 byte j-8 (j<12), high nibble of w1 byte j-12.
//   V8  8192 B  fragment F = cb*2 + kb (cb: 32-channel block, kb: 32-key block)
//               lane L byte p  <->  key kb*32 + 8*(p/4) + 4*(L/32) + p%4, channel cb*32 + L%32
//   V16 16384 B fragment F = (cb*2 + kb)*2 + kh, lane L fp16 element e (0..7)
//               <->  key kb*32 + 8*(2*kh + e/4) + 4*(L/32) + e%4, channel cb*32 + L%32
//   V4  4096 B  nibbles of the V8 layout placed as in K4 (fragment F = cb*2 + kb, so
//               16 bytes of lane L hold both 32-key blocks of channel block cb).
//
// The V orders equal the accumulator order of the QK^T MFMA (key = row of the
// 32x32 result), so a lane's probabilities feed the PV MFMA without shuffles.
#pragma once
#include <hip/hip_runtime.h>
#include <climits>
#include <stdint.h>

namespace tri {

constexpr int D = 128;
constexpr int BN = 64;
constexpr int STAT_BLOCKS = 64;
constexpr int K8_BYTES = 8192, K4_BYTES = 4096, V16_BYTES = 16384, V8_BYTES = 8192, V4_BYTES = 4096;
constexpr int KX_BYTES = 16384;            // bf16 K or V of one tile, exact heads
constexpr int K8_WORDS = K8_BYTES / 4, K4_WORDS = K4_BYTES / 4;
constexpr int V16_WORDS = V16_BYTES / 4, V8_WORDS = V8_BYTES / 4, V4_WORDS = V4_BYTES / 4;
constexpr float MAGIC = 12582912.0f;      // 1.5 * 2^23
constexpr uint32_t MAGIC_BITS = 0x4B400000u;
constexpr float PMAGIC_HALF = 49152.5f;    // P quantizer: byte 1 of fma(e, 255, 49152.5)
// Cache policy of loads that stream data read once (the decode kernels' K/V records): the
// non-temporal bit (gfx950 buffer loads, "nt"), so the stream does not displace what other loads
// reuse from the caches.  Prefill's record copies keep the default: the q-heads of a GQA group
// read the same records through L2.
constexpr int LOAD_STREAM = 2;
constexpr int MAX_TILES = 2048;            // 131072 tokens (prefill_sm80.cu:23)
constexpr int MAX_GROUP = 8;               // GQA group bound of the decode kernel
constexpr int NEAR_V8 = 16;                // decode V recency window (decode.py:9)

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  const _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

// The path's exp2: clamp to >= -125, split x = n + f with n = rint(x), 2^f = 1 + f P(f) in Horner
// order with fma, scale by 2^n.  P is the degree-5 polynomial of exp2f for 2^x on [-0.5, 0.5] in
// S. L. Moshier's Cephes Math Library (single precision), its coefficients rounded to binary32;
// evaluated so, the result is within 0.952 ulp of exp2 (every f, exhaustively).  The CPU oracle
// evaluates the identical sequence (rint, ldexp), so results agree bit for bit.
// Here n comes from the 1.5*2^23 shifter (t = x + 1.5*2^23 rounds to nearest
// even like rint, and its low mantissa bits hold n in two's complement), and
// 2^n is applied by adding n to the exponent field of p: for x in [-125, 127]
// the product is a normal float, so this equals ldexp(p, n) exactly.
__device__ __forceinline__ float texp2(float x) {
  x = fmaxf(x, -125.0f);
  const float t = x + 12582912.0f;
  const float n = t - 12582912.0f;
  const float f = x - n;
  float p = 0x1.41fbbcp-13f;
  p = __builtin_fmaf(p, f, 0x1.5f3e52p-10f);
  p = __builtin_fmaf(p, f, 0x1.3b2d4cp-7f);
  p = __builtin_fmaf(p, f, 0x1.c6aee8p-5f);
  p = __builtin_fmaf(p, f, 0x1.ebfbdcp-3f);
  p = __builtin_fmaf(p, f, 0x1.62e430p-1f);
  p = __builtin_fmaf(p, f, 1.0f);
  return __uint_as_float(__float_as_uint(p) + (__float_as_uint(t) << 23));
}

// exp2 of the prefill's per-score probabilities (P levels, fp16 P): the hardware
// v_exp_f32 (about 1 ulp), as the reference takes its per-score exp2 from the
// hardware approximation (ex2.approx.ftz.f32).  A level can differ from the
// one texp2 gives only where e * levels lies within a few ulp of a rounding
// boundary (measured: 2.6e-4 of C0's outputs move, by at most 1.5e-5; the
// prefill's PV levels are 8-bit).  texp2's polynomial costs ~10 VALU per score,
// v_exp_f32 one transcendental.  (Decode, memory-bound and with 15-level INT4
// V, takes texp2 for its levels.)
__device__ __forceinline__ float pexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Sign pattern of the 128-channel rotation (prefill_sm80.cu:95): bit c & 31 of
// word c >> 5 flips channel c.
__device__ __forceinline__ uint32_t rot_word(int w) {
  return w == 0 ? 0x9a3b5e71u : w == 1 ? 0x2c6d8f13u : w == 2 ? 0xe41b7a95u : 0x5f02c3d8u;
}
// DPP lane moves within 16-lane rows: quad_perm [1,0,3,2] (lane ^ 1), quad_perm
// [2,3,0,1] (lane ^ 2), quad_perm [3,2,1,0] (lane ^ 3), row_half_mirror (lane
// 7 - i of each 8), row_mirror (lane 15 - i of each 16).  VALU operations,
// unlike __shfl_xor's LDS permute.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// the value of lane ^ BIT, BIT in {1, 2, 4}: lane ^ 4 is the half-row mirror
// (lane ^ 7) of the quad reversal (lane ^ 3)
template <int BIT>
__device__ __forceinline__ float lane_xor8(float v) {
  if constexpr (BIT == 1) return dpp_move<0xB1>(v);
  else if constexpr (BIT == 2) return dpp_move<0x4E>(v);
  else return dpp_move<0x141>(dpp_move<0x1B>(v));
}

// one cross-lane butterfly stage over lane bit BIT of an 8-lane group
template <int BIT>
__device__ __forceinline__ void rot_stage8(float (&x)[16], int t) {
  const bool upper = t & BIT;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float y = lane_xor8<BIT>(x[i]);
    x[i] = upper ? y - x[i] : x[i] + y;
  }
}

// Rotation of one 128-vector held by 8 consecutive lanes, 16 channels each
// (channel 16*t + i in lane t of the 8-lane group), prefill_sm80.cu:95-115: sign
// flips, then butterfly stages over index bits 0..6 in order, (lo, hi) ->
// (lo + hi, lo - hi), then the 1/sqrt(128) scale.  Bits 0-3 are in-register
// stages, bits 4-6 cross-lane stages through DPP moves.
__device__ __forceinline__ void rotate128_x16(float (&x)[16], int t) {
  const uint32_t sg = rot_word(t >> 1) >> (16 * (t & 1));
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if ((sg >> i) & 1u) x[i] = -x[i];
#pragma unroll
  for (int bit = 1; bit < 16; bit <<= 1)
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (!(i & bit)) {
        const float lo = x[i], hi = x[i | bit];
        x[i] = lo + hi;
        x[i | bit] = lo - hi;
      }
  rot_stage8<1>(x, t);
  rot_stage8<2>(x, t);
  rot_stage8<4>(x, t);
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] *= 0.08838834764831845f;
}

// maximum over each group of 8 consecutive lanes
__device__ __forceinline__ float lanes8_max(float m) {
  m = fmaxf(m, lane_xor8<1>(m));
  m = fmaxf(m, lane_xor8<2>(m));
  return fmaxf(m, lane_xor8<4>(m));
}



// DPP move restricted to the 16-lane rows in ROWS; other rows keep v.  Row
// broadcasts: 0x142 (row_bcast:15) gives rows 1 and 3 lane 15 of the row before
// (with ROWS = 0xA), 0x143 (row_bcast:31) gives rows 2 and 3 lane 31 (ROWS = 0xC).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float v) {
  const int x = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(x, x, CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// maximum of each 16-lane row, in every lane of the row
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  return fmaxf(v, dpp_move<0x140>(v));
}
// maximum over the wave as a uniform value: rows, then row_bcast:15 and
// row_bcast:31 fold the rows into lane 63 (VALU only, no LDS permute)
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, dpp_rows<0x142, 0xA>(v));
  v = fmaxf(v, dpp_rows<0x143, 0xC>(v));
  return readlane_f(v, 63);
}
// maximum over the lane's 32-lane half: row_bcast:15 folds rows 0-1 into lane 31
// and rows 2-3 into lane 63
__device__ __forceinline__ float half_max(float v, bool upper) {
  v = row16_max(v);
  v = fmaxf(v, dpp_rows<0x142, 0xA>(v));
  const float lo = readlane_f(v, 31), hi = readlane_f(v, 63);
  return upper ? hi : lo;
}


// maximum of each 16-lane row of an int, in every lane of the row (the DPP moves
// fold into v_max_i32)
template <int CTRL>
__device__ __forceinline__ int dpp_move_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true);
}
__device__ __forceinline__ int row16_max_i(int v) {
  v = max(v, dpp_move_i<0xB1>(v));
  v = max(v, dpp_move_i<0x4E>(v));
  v = max(v, dpp_move_i<0x141>(v));
  return max(v, dpp_move_i<0x140>(v));
}
// maximum over the wave of a value that is uniform within each 16-lane row, as a
// uniform value: row_bcast:15 and row_bcast:31 fold the rows into lane 63
__device__ __forceinline__ float rows_max_wave(float v) {
  v = fmaxf(v, dpp_rows<0x142, 0xA>(v));
  v = fmaxf(v, dpp_rows<0x143, 0xC>(v));
  return readlane_f(v, 63);
}
// the same over the lane's 32-lane half
__device__ __forceinline__ float rows_max_half(float v, bool upper) {
  v = fmaxf(v, dpp_rows<0x142, 0xA>(v));
  const float lo = readlane_f(v, 31), hi = readlane_f(v, 63);
  return upper ? hi : lo;
}

// Lanes L and L ^ 32 combined: v_permlane32_swap hands each 32-lane half the other half's values
// (a VALU operation, no LDS round trip like __shfl_xor's permute); both halves combine the same two
// operands in the same order, so they hold identical results.
__device__ __forceinline__ void xor32_pair(uint32_t v, uint32_t& lo, uint32_t& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  lo = r[0];  // the value of lane L % 32
  hi = r[1];  // the value of lane L % 32 + 32
}
// Maxima of values that arithmetic produced (never a signaling NaN): the hardware max as is.  fmaxf
// would first canonicalize each operand that the compiler cannot trace to arithmetic (one more VALU
// operation per operand after a lane exchange or an LDS read); the results are the same.  Not for MFMA
// results: the compiler does not pad an inline-asm read of an accumulator for the MFMA's latency.
__device__ __forceinline__ float max_arith(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_arith(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float xor32_max(float v) {
  uint32_t lo, hi;
  xor32_pair(__float_as_uint(v), lo, hi);
  return max_arith(__uint_as_float(lo), __uint_as_float(hi));
}
__device__ __forceinline__ float xor32_add(float v) {
  uint32_t lo, hi;
  xor32_pair(__float_as_uint(v), lo, hi);
  return __uint_as_float(lo) + __uint_as_float(hi);
}
__device__ __forceinline__ uint32_t xor32_add(uint32_t v) {
  uint32_t lo, hi;
  xor32_pair(v, lo, hi);
  return lo + hi;
}

// byte 1 of each of four words, packed (P levels out of the 49152.5 magic).
__device__ __forceinline__ uint32_t pack_byte1(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  const uint32_t lo = __builtin_amdgcn_perm(w1, w0, 0x0c0c0501u);  // [w0.b1, w1.b1, 0, 0]
  const uint32_t hi = __builtin_amdgcn_perm(w3, w2, 0x05010c0cu);  // [0, 0, w2.b1, w3.b1]
  return lo | hi;
}

// Four packed 4-bit codes in the high halves of bytes (16 * signed code).
__device__ __forceinline__ uint32_t nib_lo16(uint32_t w) { return (w << 4) & 0xf0f0f0f0u; }
__device__ __forceinline__ uint32_t nib_hi16(uint32_t w) { return w & 0xf0f0f0f0u; }

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma_f16(v8h a, v8h b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma_bf16(v8bf a, v8bf b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace tri
