// Causal banded quantized attention for gfx950 (one launch for every q-head and
// query tile; each q-head's band picks per key tile between fp16 P x fp16 V',
// INT8 QK with u8 P x INT8 V', INT4 QK with u8 P x INT8 V', or skip).
//
// Reference semantics: triattention/kernels/cuda/prefill_sm80.cu:244-505
// (scaled_row_max, tile_base_margin, run_task, unified_kernel).
//
// Work decomposition: one workgroup of 2 waves per (batch, q-head, 64-row query
// tile); wave w owns query rows 32w..32w+31 (launches too small to give every
// SIMD a wave take 4 waves, two such pairs splitting the key tiles: PAIRS = 2
// below).  Scores are computed transposed,
// S^T = K Q^T, with v_mfma_i32_32x32x32_i8, so lane L holds the 32 scores of
// query L%32 for keys {kb*32 + 8*(r/4) + 4*(L/32) + r%4}; the same lane then
// feeds its probabilities as the B operand of O^T = V^T P^T.  Row statistics
// need one cross-lane step (lanes L and L^32 share a query).
#include "common.h"

namespace tri {

struct PrefillArgs {
  const int32_t* order;
  const int32_t* bands;
  const uint8_t* v16;
  const uint8_t* v8;
  const float* vstat;
  const int8_t* q8;
  const uint8_t* k8;
  const float* qa;
  const float* ka;
  const uint8_t* q4;
  const uint8_t* k4;
  const float* qa4;
  const float* ka4;
  void* out;
  int out_dtype;  // 0 = fp32, 1 = bf16, 2 = fp16
  int64_t osb, osh, ost;
  int hq, hk, t;
  float sm_log2;
  // exact (bf16) heads: exact[qh] = 1 + record slot of the q-head's KV head
  // (0: quantized) selects exact causal attention on the raw bf16 operands
  const int32_t* exact;
  const uint16_t* qr;
  int64_t qsb, qsh, qst;  // raw q strides (elements)
  const uint8_t* kx;      // KX records [batch][nx][tiles]
  const uint8_t* vx;      // VX records [batch][nx][tiles]
  int nx;
  // extension (may be null): per V8 record, -127 times each channel's sum of its 64 codes (int32 [128]),
  // the starting value of the tile's P V accumulators (else two MFMAs compute it)
  const int32_t* v8s;
  // extension (may be null): the INT4 K records expanded to 16 * code bytes in the INT8 record layout
  // (8 KiB per tile), which INT4 tiles then read as INT8 tiles read theirs
  const uint8_t* k4x;
};

// KQ4X: an INT4 tile whose K record is the expanded form (k4x); its arithmetic is KQ4's
enum Kind { KF16 = 0, KI8 = 1, KQ4 = 2, KQ4X = 3 };

struct PrefillState {
  v16f acc[4];     // O^T accumulators, 4 channel blocks of 32
  float m, den;    // running max (log2 units) and denominator, equal in lanes L and L^32
};

template <int KIND>
__device__ __forceinline__ v4i k_frag(const uint8_t* __restrict__ k_lds, int F, int L) {
  if constexpr (KIND == KQ4) {
    // packed 4-bit record in LDS (fragments 2P and 2P+1 share lane L's 16 bytes at
    // P*1024 + 16L): unpack this lane's 8 bytes to 16 bytes of 16*code
    const uint2 w = *reinterpret_cast<const uint2*>(k_lds + (F >> 1) * 1024 + L * 16 + (F & 1) * 8);
    return v4i{(int)nib_lo16(w.x), (int)nib_hi16(w.x), (int)nib_lo16(w.y), (int)nib_hi16(w.y)};
  } else {
    return *reinterpret_cast<const v4i*>(k_lds + F * 1024 + L * 16);
  }
}

// SUMS: the quantized P V accumulators start from the tile's -127 * sum(V8) in LDS (vs_lds, channel
// order) instead of two MFMAs against a constant -127 operand.  QMASK: a quantized tile that is the
// query tile itself (an INT4 list that reaches the diagonal, w8 = 0): keys past the query row or
// past t get level 0 and stay out of the tile max, as fp16 tiles mask them.
template <int KIND, bool SUMS = false, bool QMASK = false>
__device__ __forceinline__ void prefill_tile(const PrefillArgs& a, PrefillState& st, const v4i (&qf)[4], float qs,
                                             const float (&ks)[4], int col, bool masked, int qrow,
                                             const uint8_t* __restrict__ k_lds, const uint8_t* __restrict__ v_lds,
                                             const uint8_t* __restrict__ v_hi = nullptr,
                                             const int32_t* __restrict__ vs_lds = nullptr) {
  constexpr bool IS4 = KIND == KQ4 || KIND == KQ4X;  // INT4 arithmetic (16 * dot)
  const int L = threadIdx.x & 63, half = L >> 5;
  // ---- S^T = K Q^T over 128 features, two 32-key blocks
  v16i s[2];
  const int init = IS4 ? 0 : (int)MAGIC_BITS;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kb][r] = init;
#pragma unroll
  for (int kstep = 0; kstep < 4; ++kstep)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[kb] = mfma_i8(k_frag<KIND>(k_lds, kb * 4 + kstep, L), qf[kstep], s[kb]);

  // Under QMASK the accumulators of masked keys become INT_MIN, which no
  // accumulator reaches otherwise (8-bit: a positive float's bits; 4-bit:
  // |16 * dot| < 2^26); the max and the P levels test for it.
  if constexpr (QMASK) {
    const int lim = min(qrow, a.t - 1) - col * BN - 4 * half;  // largest valid key offset in this lane
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb * 32 + 8 * (r >> 2) + (r & 3) > lim) s[kb][r] = INT_MIN;
  }

  // score of accumulator r of block kb as a float: the magic float for 8-bit
  // codes (1.5*2^23 + dot), 16*dot for 4-bit codes (the MFMA saw 16*code keys;
  // the 1/16 is folded into the slope, which is exact).  fp16 tiles mask here.
  auto score = [&](int kb, int r) -> float {
    float v = IS4 ? (float)s[kb][r] : __int_as_float(s[kb][r]);
    if constexpr (KIND == KF16) {
      if (masked) {
        const int key = col * BN + kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (key > qrow || key >= a.t) v = -__builtin_inff();
      }
    }
    return v;
  };

  // ---- scaled row max (prefill_sm80.cu:244-253)
  float slope[4];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) slope[gi] = IS4 ? qs * ks[gi] * 0.0625f : qs * ks[gi];
  float tile = -__builtin_inff();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int hg = 0; hg < 2; ++hg) {
      if constexpr (KIND == KF16) {
        float mx = score(kb, hg * 8);
#pragma unroll
        for (int r = 1; r < 8; ++r) mx = fmaxf(mx, score(kb, hg * 8 + r));
        if (mx > -__builtin_inff()) tile = fmaxf(tile, slope[kb * 2 + hg] * (mx - MAGIC));
      } else {
        // the group's largest integer accumulator (the magic-offset dot product, or 16 * dot), whose
        // order is the scores' order, converted once (under QMASK a group with no valid key, all
        // INT_MIN, leaves the tile max alone)
        const int g0 = hg * 8;
        int mx = max(max(s[kb][g0], s[kb][g0 + 1]), s[kb][g0 + 2]);
        mx = max(max(mx, s[kb][g0 + 3]), s[kb][g0 + 4]);
        mx = max(max(mx, s[kb][g0 + 5]), s[kb][g0 + 6]);
        mx = max(mx, s[kb][g0 + 7]);
        // (|dot| < 2^22: the magic float minus 1.5 * 2^23 is the dot product exactly)
        const float d = IS4 ? (float)mx : __int_as_float(mx) - MAGIC;
        if (!QMASK || mx != INT_MIN) tile = fmaxf(tile, slope[kb * 2 + hg] * d);
      }
    }
  tile = xor32_max(tile);
  // Running reference max.  fp16 tiles need the exact running max (their P
  // is relative to it).  INT8/INT4 P levels are relative to the tile's own
  // base, so the reference max only scales acc and den alike and acc/den does
  // not depend on it: those tiles move it only when a tile exceeds it by more
  // than 64, which skips most rescales.  Headroom: bq <= 2^(64 + margin)/255
  // and |PV| < 2^21 per tile, so acc stays below 2^(64 + 21 + 11) over 2048
  // tiles, far inside fp32.
  const float n = KIND == KF16 ? fmaxf(st.m, tile) : (tile > st.m + 64.f ? tile : st.m);
  // (quantized tiles rarely move the max: the factor and the rescale only when some row's does)
  float alpha = 1.f;
  if (KIND == KF16 || __any(n != st.m)) alpha = texp2(st.m - n);
  st.m = n;
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[cb][r] *= alpha;
  }

  if constexpr (KIND == KF16) {
    // ---- fp16 P x fp16 V' (prefill_sm80.cu:358-383)
    st.den *= alpha;
    float c[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) c[gi] = __builtin_fmaf(-slope[gi], MAGIC, -st.m);
    v8h p[2][2];
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gi = kb * 2 + (r >> 3);
        // (a zero query row has slope 0, and 0 * -inf of a masked key is NaN: the clamp turns it
        // into 2^-125, which rounds to fp16 0 as the masked key's probability must)
        const _Float16 h = (_Float16)pexp2(fmaxf(__builtin_fmaf(slope[gi], score(kb, r), c[gi]), -125.f));
        p[kb][r >> 3][r & 7] = h;
        psum += (float)h;
      }
    st.den += xor32_add(psum);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          // fp16 V record: fragments 0..7 in v_lds, 8..15 in v_hi
          const int F = (cb * 2 + kb) * 2 + kh;
          const v8h vf = *reinterpret_cast<const v8h*>((F < 8 ? v_lds : v_hi) + (F & 7) * 1024 + L * 16);
          st.acc[cb] = mfma_f16(vf, p[kb][kh], st.acc[cb]);
        }
  } else {
    // ---- quantized P (u8) x INT8 V' (prefill_sm80.cu:384-449)
    const float ksmax = max_arith(max3_arith(ks[0], ks[1], ks[2]), ks[3]);
    float base = tile > -__builtin_inff() ? tile : st.m;
    base += __builtin_fmaf(qs * ksmax, 0.75f, fabsf(base) * 2.4e-7f);
    // the reference divides by the level count under fast math; here: times its rounded reciprocal
    const float bq = texp2(base - st.m) * (1.f / 255.f);
    float c[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi)
      c[gi] = KIND == KI8 ? __builtin_fmaf(-slope[gi], MAGIC, -base) : -base;
    uint32_t pw[2][4];
    int rsn = 0;  // sum of this lane's 32 bytes 127 - P (signed dot product of the s8 operand words)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        uint32_t y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = qd * 4 + i, gi = kb * 2 + (r >> 3);
          float e = pexp2(__builtin_fmaf(slope[gi], score(kb, r), c[gi]));
          if constexpr (QMASK) e = s[kb][r] == INT_MIN ? 0.f : e;
          y[i] = __float_as_uint(__builtin_fmaf(e, 255.f, PMAGIC_HALF));
        }
        pw[kb][qd] = pack_byte1(y[0], y[1], y[2], y[3]) ^ 0x7f7f7f7fu;  // 127 - P as s8
        rsn = __builtin_amdgcn_sdot4((int)pw[kb][qd], 0x01010101, rsn, false);
      }
    // the row's 64 levels: 2 * 32 * 127 minus the sum of 127 - P over lanes L and L ^ 32 (mod 2^32)
    const uint32_t rs = 8128u - xor32_add((uint32_t)rsn);
    st.den = __builtin_fmaf((float)rs, bq, st.den * alpha);
    const v4i neg127 = {(int)0x81818181u, (int)0x81818181u, (int)0x81818181u, (int)0x81818181u};
    const v4i b0 = {(int)pw[0][0], (int)pw[0][1], (int)pw[0][2], (int)pw[0][3]};
    const v4i b1 = {(int)pw[1][0], (int)pw[1][1], (int)pw[1][2], (int)pw[1][3]};
    const float nbq = -bq;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const v4i va = *reinterpret_cast<const v4i*>(v_lds + (cb * 2 + 0) * 1024 + L * 16);
      const v4i vb = *reinterpret_cast<const v4i*>(v_lds + (cb * 2 + 1) * 1024 + L * 16);
      v16i d = {};
      if constexpr (SUMS) {
        // accumulator r of channel block cb is channel cb*32 + 8*(r/4) + 4*half + r%4
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v4i w = *reinterpret_cast<const v4i*>(vs_lds + cb * 32 + 8 * j + 4 * half);
#pragma unroll
          for (int i = 0; i < 4; ++i) d[4 * j + i] = w[i];
        }
      } else {
        d = mfma_i8(va, neg127, d);
        d = mfma_i8(vb, neg127, d);
      }
      d = mfma_i8(va, b0, d);
      d = mfma_i8(vb, b1, d);  // = -sum_k P_k v_k
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[cb][r] = __builtin_fmaf((float)d[r], nbq, st.acc[cb][r]);
    }
  }
}

// Asynchronous global -> LDS copy of BYTES (a multiple of 2 KiB) by the two
// waves of the workgroup, 1 KiB per wave instruction (lane L's 16 bytes land
// at dst + 16 L); completion is awaited with s_waitcnt + barrier.  The wave
// index is uniform, so src + off stays in scalar registers and each copy is
// one instruction with a 32-bit lane offset.
template <int BYTES>
__device__ __forceinline__ void lds_copy_async(const uint8_t* src, uint8_t* dst) {
  static_assert(BYTES % 2048 == 0, "copies move 2 KiB per step");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = (threadIdx.x & 63) * 16;
#pragma unroll
  for (int i = 0; i < BYTES / 2048; ++i) {
    const int off = i * 2048 + wave * 1024;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + off + lane),
                                     (__attribute__((address_space(3))) void*)(dst + off), 16, 0, 0);
  }
}

// The same copy from a buffer resource at byte offset soff (uniform), wave w
// moving the w-th half of the record (whalf = w * BYTES / 2, computed once per
// kernel): one LDS base (M0) and one scalar offset per record and wave, the
// 1 KiB steps in the instruction's offset field, which moves the global and
// the LDS address alike.
template <int BYTES>
__device__ __forceinline__ void lds_copy_buf(__amdgpu_buffer_rsrc_t src, int soff, uint8_t* dst, int whalf) {
  static_assert(BYTES == 4096 || BYTES == 8192, "records of 4 or 8 KiB");
  const int lane = (threadIdx.x & 63) * 16;
  auto* d = (__attribute__((address_space(3))) void*)(dst + whalf);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(src, d, 16, lane, soff + whalf, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(src, d, 16, lane, soff + whalf, 1024, 0);
  if constexpr (BYTES == 8192) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src, d, 16, lane, soff + whalf, 2048, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src, d, 16, lane, soff + whalf, 3072, 0);
  }
}

__device__ __forceinline__ void lds_wait() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Exact attention of one (q-head, 64-row query tile) on the raw bf16 operands:
// bf16 MFMA for QK^T (fp32 accumulation), fp32 online softmax in log2 units,
// P split into bf16 high and low parts so that P V keeps ~2^-17 relative
// precision, fp32 accumulation.  The reference's "exact" attention is
// scaled_dot_product_attention over bf16 q/k/v (triattention/models.py:45-47).
//
// Keys stream in 32-key steps: step s covers half kb = s & 1 of tile s >> 1,
// whose K and V records are 8 KiB each (KX/VX layouts below) and land in the
// LDS buffers of parity kb while step s - 1 computes.
template <bool MASKED>
__device__ __forceinline__ void exact_step(const PrefillArgs& a, int col, int kb, int qrow, const v8bf (&qf)[8],
                                           v16f (&acc)[4], float& m, float& den, const uint8_t* __restrict__ kl,
                                           const uint8_t* __restrict__ vl) {
  const int L = threadIdx.x & 63, half = L >> 5;
  // S^T = K Q^T for 32 keys x 32 queries
  v16f s = {};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
    s = mfma_bf16(*reinterpret_cast<const v8bf*>(kl + ks * 1024 + L * 16), qf[ks], s);
  if constexpr (MASKED) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = col * BN + kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
      if (key > qrow || key >= a.t) s[r] = -__builtin_inff();
    }
  }
  // row max on the raw dot products (the scale is positive), in log2 units after
  float mx = s[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
  mx = xor32_max(mx);
  const float tile = mx * a.sm_log2;
  // Reference max for P = 2^(x - m): acc and den scale alike, so m only needs
  // to keep P in range; it moves when a step exceeds it by more than 16.
  const float n = tile > m + 16.f ? tile : m;
  if (n != m) {
    const float alpha = __builtin_amdgcn_exp2f(m - n);
    m = n;
    den *= alpha;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cb][r] *= alpha;
    }
  }
  // P in pairs: one packed conversion gives the two high parts, their fp32 values are the high
  // and low halves of that word, and a second packed conversion gives the two low parts
  uint32_t hw[8], lw[8];
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * j], a.sm_log2, -m));
    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * j + 1], a.sm_log2, -m));
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){p0, p1}, v2bf));
    const float h0 = __uint_as_float(h << 16), h1 = __uint_as_float(h & 0xffff0000u);
    hw[j] = h;
    lw[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){p0 - h0, p1 - h1}, v2bf));
    psum += p0;
    psum += p1;
  }
  const v8bf phi[2] = {__builtin_bit_cast(v8bf, make_uint4(hw[0], hw[1], hw[2], hw[3])),
                       __builtin_bit_cast(v8bf, make_uint4(hw[4], hw[5], hw[6], hw[7]))};
  const v8bf plo[2] = {__builtin_bit_cast(v8bf, make_uint4(lw[0], lw[1], lw[2], lw[3])),
                       __builtin_bit_cast(v8bf, make_uint4(lw[4], lw[5], lw[6], lw[7]))};
  den += xor32_add(psum);
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const v8bf vf = *reinterpret_cast<const v8bf*>(vl + (cb * 2 + kh) * 1024 + L * 16);
      acc[cb] = mfma_bf16(vf, phi[kh], acc[cb]);
      acc[cb] = mfma_bf16(vf, plo[kh], acc[cb]);
    }
}

__device__ __forceinline__ void prefill_exact(const PrefillArgs& a, int b, int qh, int qb, uint8_t* k0, uint8_t* k1,
                                              uint8_t* v0, uint8_t* v1) {
  const int tiles = (a.t + BN - 1) / BN;
  const int tid = threadIdx.x, wave = tid >> 6, L = tid & 63, lq = L & 31, half = L >> 5;
  const int qrow = qb * BN + wave * 32 + lq;
  const bool row_ok = qrow < a.t;
  v8bf qf[8];
  const uint16_t* qp = a.qr + b * a.qsb + qh * a.qsh + (int64_t)(row_ok ? qrow : 0) * a.qst;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    // (a conditional load, not a select between the row and a zero: a select of the two addresses
    // would put the zero in scratch memory and make the load a flat one)
    uint4 w = make_uint4(0, 0, 0, 0);
    if (row_ok) w = *reinterpret_cast<const uint4*>(qp + ks * 16 + 8 * half);
    qf[ks] = __builtin_bit_cast(v8bf, w);
  }
  const int64_t rec0 = ((int64_t)b * a.nx + (a.exact[qh] - 1)) * tiles;
  const uint8_t* kx = a.kx + rec0 * KX_BYTES;
  const uint8_t* vx = a.vx + rec0 * KX_BYTES;
  v16f acc[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[cb][r] = 0.f;
  float m = -3.402823466e38f, den = 0.f;
  // the head's records as buffer resources: step st at byte (st / 2) * KX_BYTES + (st % 2) * KX_BYTES / 2
  const __amdgpu_buffer_rsrc_t rkx =
      __builtin_amdgcn_make_buffer_rsrc((void*)kx, (short)0, tiles * KX_BYTES, 0x00020000);
  const __amdgpu_buffer_rsrc_t rvx =
      __builtin_amdgcn_make_buffer_rsrc((void*)vx, (short)0, tiles * KX_BYTES, 0x00020000);
  const int whalf = __builtin_amdgcn_readfirstlane(wave) * (KX_BYTES / 4);
  auto issue = [&](int st, uint8_t* kd, uint8_t* vd) {
    const int off = (st >> 1) * KX_BYTES + (st & 1) * (KX_BYTES / 2);
    lds_copy_buf<KX_BYTES / 2>(rkx, off, kd, whalf);
    lds_copy_buf<KX_BYTES / 2>(rvx, off, vd, whalf);
  };
  issue(0, k0, v0);
  // tiles before the diagonal: no mask
  for (int col = 0; col < qb; ++col) {
    lds_wait();  // half 0 of tile col landed; every wave is done with half 1 of tile col-1
    issue(2 * col + 1, k1, v1);
    exact_step<false>(a, col, 0, qrow, qf, acc, m, den, k0, v0);
    lds_wait();  // half 1 landed; every wave is done with half 0
    issue(2 * col + 2, k0, v0);
    exact_step<false>(a, col, 1, qrow, qf, acc, m, den, k1, v1);
  }
  // the diagonal tile qb, masked
  lds_wait();
  issue(2 * qb + 1, k1, v1);
  exact_step<true>(a, qb, 0, qrow, qf, acc, m, den, k0, v0);
  lds_wait();
  exact_step<true>(a, qb, 1, qrow, qf, acc, m, den, k1, v1);
  if (!row_ok) return;
  const float inv = 1.f / den;
  const int64_t obase = b * a.osb + qh * a.osh + (int64_t)qrow * a.ost;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int ch = cb * 32 + 8 * r4 + 4 * half;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = acc[cb][r4 * 4 + i] * inv;
      if (a.out_dtype == 0) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase + ch) = make_float4(v[0], v[1], v[2], v[3]);
      } else if (a.out_dtype == 1) {
        const uint32_t lo = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
        const uint32_t hi = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase + ch) = make_uint2(lo, hi);
      } else {
        const uint32_t lo = f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16);
        const uint32_t hi = f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase + ch) = make_uint2(lo, hi);
      }
    }
}

// Packs the K and V of every exact KV head into KX / VX records (one workgroup
// per (tile, KV head, sequence); other heads return at once).  Keys at or past
// t are zero.  Per 64-key tile, 16 KiB each, 32-key half kb at byte kb*8192:
//   KX fragment F = ks (16-feature step), lane L 16 bytes = bf16 K[key kb*32 + L%32]
//      [features ks*16 + 8*(L/32) .. +7]      (A operand of S^T = K Q^T)
//   VX fragment F = cb*2 + kh, lane L element e = bf16 V[key kb*32 + 16*kh + 8*(e/4)
//      + 4*(L/32) + e%4][channel cb*32 + L%32] (A operand of O^T = V^T P^T)
struct ExactPackArgs {
  const uint16_t* k;
  const uint16_t* v;
  int64_t ksb, ksh, kst, vsb, vsh, vst;
  const int32_t* exact;  // [hq]: 1 + record slot of the q-head's KV head, 0 if quantized
  uint8_t* kx;
  uint8_t* vx;
  int hq, hk, t, nx;
};

// One tile of pack_exact: keys r < rows of ksrc / vsrc (row strides kst / vst) into the KX and VX
// records kd / vd; vt is the workgroup's LDS staging of V.  256 threads.
constexpr int EXACT_VP = D + 8;  // padded LDS row of the V staging (bf16 elements)
__device__ __forceinline__ void pack_exact_tile(const uint16_t* ksrc, int64_t kst, const uint16_t* vsrc, int64_t vst,
                                                int rows, uint8_t* kd, uint8_t* vd, uint16_t* vt) {
  const int tid = threadIdx.x;
  // K: 1024 16-byte pieces in source order (key, 8-feature piece)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, key = c >> 4, f0 = (c & 15) * 8;
    uint4 w = make_uint4(0, 0, 0, 0), u = w;
    if (key < rows) {
      w = *reinterpret_cast<const uint4*>(ksrc + (int64_t)key * kst + f0);
      u = *reinterpret_cast<const uint4*>(vsrc + (int64_t)key * vst + f0);
    }
    const int kb = key >> 5, lk = key & 31, ks = f0 >> 4, h = (f0 >> 3) & 1;
    *reinterpret_cast<uint4*>(kd + kb * (KX_BYTES / 2) + ks * 1024 + (h * 32 + lk) * 16) = w;
    *reinterpret_cast<uint4*>(vt + key * EXACT_VP + f0) = u;
  }
  __syncthreads();
  // V: 1024 output pieces in destination order
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, F = c >> 6, L = c & 63;  // F = kb*8 + cb*2 + kh
    const int kb = F >> 3, cb = (F >> 1) & 3, khalf = F & 1, ch = cb * 32 + (L & 31), h = L >> 5;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e0 = 2 * j, e1 = 2 * j + 1;
      const int k0 = kb * 32 + 16 * khalf + 8 * (e0 >> 2) + 4 * h + (e0 & 3);
      const int k1 = kb * 32 + 16 * khalf + 8 * (e1 >> 2) + 4 * h + (e1 & 3);
      w[j] = (uint32_t)vt[k0 * EXACT_VP + ch] | ((uint32_t)vt[k1 * EXACT_VP + ch] << 16);
    }
    *reinterpret_cast<uint4*>(vd + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__global__ __launch_bounds__(256) void pack_exact_kernel(ExactPackArgs a) {
  const int tile = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int slot = a.exact[kh * (a.hq / a.hk)] - 1;
  if (slot < 0) return;
  const int tiles = gridDim.x;
  const int64_t rec = ((int64_t)b * a.nx + slot) * tiles + tile;
  __shared__ __align__(16) uint16_t vt[BN * EXACT_VP];
  pack_exact_tile(a.k + b * a.ksb + kh * a.ksh + (int64_t)tile * BN * a.kst, a.kst,
                  a.v + b * a.vsb + kh * a.vsh + (int64_t)tile * BN * a.vst, a.vst, a.t - tile * BN,
                  a.kx + rec * KX_BYTES, a.vx + rec * KX_BYTES, vt);
}

template <int V>
struct Tag {
  static constexpr int value = V;
};

// SUMS: a.v8s is given (the P V accumulators of quantized tiles start from it).
// PAIRS = 2 (launches with too few workgroups to give every SIMD a wave): four
// waves per workgroup, two pairs over the same 64 query rows; pair 0 takes the
// F16 tiles and the first part of the quantized tile list, pair 1 the rest,
// each with LDS buffers of its own, and pair 0 merges pair 1's running state
// (max, denominator, accumulators) through LDS before the epilogue.  Every wave
// passes the same number of barriers (the pair with fewer tiles waits out the
// difference), as a workgroup barrier counts the arrivals of all four.
template <bool SUMS, int PAIRS>
__global__ __launch_bounds__(128 * PAIRS) __attribute__((amdgpu_waves_per_eu(2))) void prefill_kernel(PrefillArgs a) {
  // LDS: two K buffers (8 KiB) and two V buffers (8 KiB) per pair, distinct
  // objects so that the compiler can tell a read of one buffer from a load into
  // the other; an fp16 V record uses both V buffers
  __shared__ __align__(16) uint8_t k_lds0[PAIRS][K8_BYTES], k_lds1[PAIRS][K8_BYTES];
  __shared__ __align__(16) uint8_t v_lds0[PAIRS][V8_BYTES], v_lds1[PAIRS][V8_BYTES];
  // the tile's -127 * V8 sums (D words, with SUMS) followed by its 4 K group scales as an INT8 tile
  // and as an INT4 tile, which one copy instruction brings together
  constexpr int VK = SUMS ? D : 0;
  __shared__ __align__(16) int32_t vk_lds0[PAIRS][VK + 8], vk_lds1[PAIRS][VK + 8];
  __shared__ __align__(16) float vms_lds[2 * D];  // the KV head's V mean and scale, for the epilogue
  const int rows = (a.t + BN - 1) / BN;
  // Launch sequence: BandTable's order is KV-head-major (prefill.py:24-25), so the workgroups running at
  // any one time would all belong to one KV head.  Group t of the sequence is query tile qd = t / hk of
  // KV head kv = t % hk, and its q-head r takes entry (kv * rows + qd) * g + r: the same entries,
  // longest query tiles still first, but the KV heads interleaved, so exact heads (MFMA-heavy) run
  // beside quantized ones (VALU-heavy) on the same CUs.  The group's q-heads read the same K/V tiles:
  // when the groups fill whole rounds of the 8 XCDs (which receive the workgroups round-robin, XCD =
  // blockIdx.x % 8 as gridDim.x is then a multiple of 8), XCD x's k-th workgroup, blockIdx.x = 8k + x,
  // is q-head k % g of group 8 (k / g) + (x + k / g) % 8, so that a group's q-heads share one XCD's L2
  // and each XCD still moves through the KV heads.
  int j = blockIdx.x;
  if ((int)gridDim.x == a.hq * rows) {
    const int g0 = a.hq / a.hk;
    int r = j % g0, t = j / g0;
    if ((a.hk * rows) % 8 == 0) {
      const int x = j & 7, k = j >> 3, gk = k / g0;
      r = k % g0;
      t = gk * 8 + ((x + gk) & 7);
    }
    j = ((t % a.hk) * rows + t / a.hk) * g0 + r;
  }
  const int task = __builtin_amdgcn_readfirstlane(a.order[j]), b = blockIdx.y;
  const int qh = task / rows, qb = task % rows, g = a.hq / a.hk, kh = qh / g;
  const int pair = PAIRS == 2 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 7)) : 0;
  if (a.exact != nullptr && a.exact[qh] > 0) {
    // (pair 0 alone; pair 1 passes the exact path's two barriers per key tile)
    if (pair == 0) prefill_exact(a, b, qh, qb, k_lds0[0], k_lds1[0], v_lds0[0], v_lds1[0]);
    else
      for (int k = 0; k < 2 * (qb + 1); ++k) __syncthreads();
    return;
  }
  const int tid = threadIdx.x & 127, wave = tid >> 6, L = tid & 63, lq = L & 31, half = L >> 5;
  const int qrow = qb * BN + wave * 32 + lq;
  const bool row_ok = qrow < a.t;
  const int tiles = rows;
  const int64_t qrow_idx = ((int64_t)b * a.hq + qh) * a.t + qrow;
  const int64_t rec0 = ((int64_t)b * a.hk + kh) * tiles;

  // band lists (prefill_sm80.cu:280-286)
  const int w8 = a.bands[2 * qh], w4 = a.bands[2 * qh + 1];
  const int lo8 = max(1, qb - w8 + 1), n8 = max(0, qb - lo8);
  const int lo4 = max(1, qb - w4 + 1), n4 = max(0, qb - w8 - lo4 + 1);

  v4i qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    qf[ks] = v4i{0, 0, 0, 0};
    if (row_ok) qf[ks] = *reinterpret_cast<const v4i*>(a.q8 + qrow_idx * D + ks * 32 + 16 * half);
  }
  const float qs8 = row_ok ? a.qa[qrow_idx] * a.sm_log2 : 1.17549435e-38f;
  PrefillState st;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.acc[cb][r] = 0.f;
  st.m = -3.402823466e38f;
  st.den = 0.f;
  const float* ka8 = a.ka + rec0 * 4;
  const float* ka4p = a.ka4 ? a.ka4 + rec0 * 4 : nullptr;

  // ---- F16 pass: tile 0, then the diagonal tile when qb > 0 (synchronous staging; pair 0)
  const int nf16 = qb > 0 ? 2 : 1;
  // this pair's part [q0, q1) of the quantized tile list (INT8 tiles, then INT4 ones): with two pairs,
  // pair 0's F16 tiles (each priced as two quantized ones: their copies are synchronous) and quantized
  // tiles balance pair 1's (C0 attention: 25.3 us with the F16 tiles priced as one, 23.6 as two, 24.9
  // as three)
  const int total = n8 + n4;
  const int c = PAIRS == 2 ? max(0, (total - 2 * nf16 + 1) / 2) : total;
  const int q0 = pair == 0 ? 0 : c, q1 = pair == 0 ? c : total;
  // barriers each pair passes: two per F16 tile, one before its quantized part and one per tile of it
  const int bar0 = 2 * nf16 + (c > 0 ? 1 + c : 0), bar1 = total > c ? 1 + total - c : 0;
  for (int i = 0; i < (pair == 0 ? nf16 : 0); ++i) {
    const int col = i == 0 ? 0 : qb;
    __syncthreads();
    // (with the first copy: the epilogue's V mean and scale, 1 KiB, so that it reads them from LDS)
    if (i == 0 && tid < 64)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(a.vstat + ((int64_t)b * a.hk + kh) * 3 * D + tid * 4),
                                       (__attribute__((address_space(3))) void*)(vms_lds + tid * 4), 16, 0, 0);
    lds_copy_async<K8_BYTES>(a.k8 + (rec0 + col) * K8_BYTES, k_lds0[0]);
    lds_copy_async<V16_BYTES / 2>(a.v16 + (rec0 + col) * V16_BYTES, v_lds0[0]);
    lds_copy_async<V16_BYTES / 2>(a.v16 + (rec0 + col) * V16_BYTES + V16_BYTES / 2, v_lds1[0]);
    lds_wait();
    const float ks[4] = {ka8[col * 4], ka8[col * 4 + 1], ka8[col * 4 + 2], ka8[col * 4 + 3]};
    prefill_tile<KF16>(a, st, qf, qs8, ks, col, i == nf16 - 1 && col == qb, qrow, k_lds0[0], v_lds0[0], v_lds1[0]);
  }

  // ---- INT8 then INT4 passes as one pipelined tile list: the next tile's
  // records stream into the other LDS buffer while the current one is used
  if (q0 < q1) {
    v4i q4f[4];
    float qs4 = 1.17549435e-38f;
    if (n4 > 0) {
      // INT4 Q codes, sign-extended to bytes in feature order
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        uint2 raw = make_uint2(0u, 0u);
        if (row_ok) raw = *reinterpret_cast<const uint2*>(a.q4 + qrow_idx * (D / 2) + (ks * 32 + 16 * half) / 2);
        const uint32_t wd[2] = {raw.x, raw.y};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = wd[j >> 1] >> (16 * (j & 1));
          uint32_t out = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t nib = (w >> (4 * e)) & 0xfu;
            out |= ((uint32_t)(((int)(nib ^ 8u)) - 8) & 0xffu) << (8 * e);
          }
          o[j] = out;
        }
        q4f[ks] = v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      }
      if (row_ok) qs4 = a.qa4[qrow_idx] * a.sm_log2;
    }
    auto tile_col = [&](int i) { return i < n8 ? lo8 + i : lo4 + (i - n8); };
    // the (sequence, KV head)'s record ranges as buffer resources: tile col at byte col * size
    const __amdgpu_buffer_rsrc_t rk8 =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.k8 + rec0 * K8_BYTES), (short)0, tiles * K8_BYTES, 0x00020000);
    const __amdgpu_buffer_rsrc_t rk4 = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.k4 ? a.k4 + rec0 * K4_BYTES : a.k8), (short)0, a.k4 ? tiles * K4_BYTES : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv8 =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.v8 + rec0 * V8_BYTES), (short)0, tiles * V8_BYTES, 0x00020000);
    const bool k4x = a.k4x != nullptr;  // INT4 tiles read the expanded records (8 KiB each)
    const __amdgpu_buffer_rsrc_t rk4x = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(k4x ? a.k4x + rec0 * K8_BYTES : a.k8), (short)0, k4x ? tiles * K8_BYTES : 0, 0x00020000);
    // (a local copy: reading the kernel argument inside the lambda would put the argument block in
    // private memory)
    const int32_t* v8s = SUMS ? a.v8s + rec0 * D : nullptr;
    // each wave's half of a record (the copies' per-wave offsets, uniform)
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int kh8 = wv * (K8_BYTES / 2), kh4 = wv * (K4_BYTES / 2), vh8 = wv * (V8_BYTES / 2);
    // The tile's V8 sums and both lists' K scales in one instruction of wave 0: lanes 0..31 copy 16
    // bytes of sums each (with SUMS), the next lane the INT8 list's scales and the one after it the
    // INT4 list's (at words VK and VK + 4), each lane from its own base and stride, so that reading
    // them later waits on nothing but the records' own wait.
    const int nsmall = VK / 4 + 2;
    const uint8_t* sbase = nullptr;
    int sshift = 4;
    if (tid < nsmall) {
      if (SUMS && tid < 32) {
        sbase = reinterpret_cast<const uint8_t*>(v8s) + tid * 16;
        sshift = 9;  // D int32 words per tile
      } else {
        sbase = reinterpret_cast<const uint8_t*>(tid == VK / 4 || ka4p == nullptr ? ka8 : ka4p);
      }
    }
    auto issue_small = [&](int col, int32_t* vkd) __attribute__((always_inline)) {
      if (tid < nsmall)
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(sbase + ((int64_t)col << sshift)),
                                         (__attribute__((address_space(3))) void*)vkd, 16, 0, 0);
    };
    // Tile i's copies when it is of kind K (its K records: INT8, expanded INT4 or packed INT4), so
    // that an INT4 loop issues its next tile's copies with no branch on the format.
    auto issue_as = [&](auto kind, int i, uint8_t* kd, uint8_t* vd, int32_t* vkd) __attribute__((always_inline)) {
      constexpr int K = decltype(kind)::value;
      const int col = K == KI8 ? lo8 + i : lo4 + (i - n8);
      if constexpr (K == KI8) lds_copy_buf<K8_BYTES>(rk8, col * K8_BYTES, kd, kh8);
      else if constexpr (K == KQ4X) lds_copy_buf<K8_BYTES>(rk4x, col * K8_BYTES, kd, kh8);
      else lds_copy_buf<K4_BYTES>(rk4, col * K4_BYTES, kd, kh4);
      lds_copy_buf<V8_BYTES>(rv8, col * V8_BYTES, vd, vh8);
      issue_small(col, vkd);
    };
    // tile i of either list, i < total (the INT8 loop's next tile may start the INT4 list): the
    // expanded or INT8 K record of the same size from a selected resource, branching only for the
    // packed INT4 form of a reference-shaped call
    auto issue = [&](int i, uint8_t* kd, uint8_t* vd, int32_t* vkd) __attribute__((always_inline)) {
      const bool is8 = i < n8;
      const int col = is8 ? lo8 + i : lo4 + (i - n8);
      if (is8 || k4x) lds_copy_buf<K8_BYTES>(is8 ? rk8 : rk4x, col * K8_BYTES, kd, kh8);
      else lds_copy_buf<K4_BYTES>(rk4, col * K4_BYTES, kd, kh4);
      lds_copy_buf<V8_BYTES>(rv8, col * V8_BYTES, vd, vh8);
      issue_small(col, vkd);
    };
    // tile i of kind KIND: wait for its records (and for every wave to finish
    // tile i-1, whose buffers receive tile i+1), start tile i+1's loads, compute
    auto step = [&](auto kind, auto mask, int i, const uint8_t* kc, const uint8_t* vc, const int32_t* vkc,
                    uint8_t* kn, uint8_t* vn, int32_t* vkn) __attribute__((always_inline)) {
      lds_wait();
      constexpr int KIND = decltype(kind)::value;
      if (i + 1 < q1) {
        // an INT4 tile is followed by one of its own kind, an INT8 tile by INT8 up to the list's end
        if constexpr (KIND == KI8) issue(i + 1, kn, vn, vkn);
        else issue_as(kind, i + 1, kn, vn, vkn);
      }
      const int col = tile_col(i);
      const float4 k4v = *reinterpret_cast<const float4*>(vkc + VK + (KIND == KI8 ? 0 : 4));
      const float ks[4] = {k4v.x, k4v.y, k4v.z, k4v.w};
      constexpr bool QMASK = decltype(mask)::value != 0;
      if constexpr (KIND == KI8) prefill_tile<KI8, SUMS>(a, st, qf, qs8, ks, col, false, qrow, kc, vc, nullptr, vkc);
      else prefill_tile<KIND, SUMS, QMASK>(a, st, q4f, qs4, ks, col, QMASK, qrow, kc, vc, nullptr, vkc);
    };
    // Tiles [i, end) of one kind, the first in buffer set PARITY.  Each kind has a
    // loop of its own: with both kinds in one loop body the compiler copies the
    // accumulators between register sets at every tile (~30 VALU per tile).
    auto run = [&](auto kind, auto parity, int i, int end) __attribute__((always_inline)) {
      constexpr bool p = decltype(parity)::value != 0;
      uint8_t* k0 = p ? k_lds1[pair] : k_lds0[pair];
      uint8_t* k1 = p ? k_lds0[pair] : k_lds1[pair];
      uint8_t* v0 = p ? v_lds1[pair] : v_lds0[pair];
      uint8_t* v1 = p ? v_lds0[pair] : v_lds1[pair];
      int32_t* w0 = p ? vk_lds1[pair] : vk_lds0[pair];
      int32_t* w1 = p ? vk_lds0[pair] : vk_lds1[pair];
      for (; i < end; i += 2) {
        step(kind, Tag<0>{}, i, k0, v0, w0, k1, v1, w1);
        if (i + 1 < end) step(kind, Tag<0>{}, i + 1, k1, v1, w1, k0, v0, w0);
      }
    };
    // The INT4 list ends at the query tile itself when w8 = 0 (then n8 = 0): that last tile is
    // masked like the reference masks the last entry of a pass when it is the query tile
    // (prefill_sm80.cu:328-329), in a step of its own outside the loop.
    // (the list's last tile, which the last part holds)
    const bool diag4 = w8 <= 0 && n4 > 0 && q1 == total;
    const int s4 = max(n8, q0), end4 = q1 - (diag4 ? 1 : 0);
    auto last = [&](auto kind) __attribute__((always_inline)) {
      if (!diag4) return;
      if ((total - 1 - q0) & 1)
        step(kind, Tag<1>{}, total - 1, k_lds1[pair], v_lds1[pair], vk_lds1[pair], k_lds0[pair], v_lds0[pair],
             vk_lds0[pair]);
      else
        step(kind, Tag<1>{}, total - 1, k_lds0[pair], v_lds0[pair], vk_lds0[pair], k_lds1[pair], v_lds1[pair],
             vk_lds1[pair]);
    };
    __syncthreads();  // every wave is done with the F16 pass's LDS
    issue(q0, k_lds0[pair], v_lds0[pair], vk_lds0[pair]);
    run(Tag<KI8>{}, Tag<0>{}, q0, min(n8, q1));
    if (k4x) {
      if ((s4 - q0) & 1) run(Tag<KQ4X>{}, Tag<1>{}, s4, end4);
      else run(Tag<KQ4X>{}, Tag<0>{}, s4, end4);
      last(Tag<KQ4X>{});
    } else {
      if ((s4 - q0) & 1) run(Tag<KQ4>{}, Tag<1>{}, s4, end4);
      else run(Tag<KQ4>{}, Tag<0>{}, s4, end4);
      last(Tag<KQ4>{});
    }
  }

  if constexpr (PAIRS == 2) {
    // the pair with fewer barriers waits out the difference
    for (int k = pair == 0 ? bar0 : bar1; k < max(bar0, bar1); ++k) __syncthreads();
    // (each pair's last barrier came before its last tile: wait until every wave is done with its buffers)
    __syncthreads();
    // pair 1's running state through LDS (over the K and V buffers, which every wave is done with):
    // wave w's accumulators in one 16 KiB object, element-major, lane-minor; the maxima and
    // denominators after them in another
    float* xs = reinterpret_cast<float*>(wave == 0 ? &k_lds0[0][0] : &k_lds1[0][0]);
    float* ms = reinterpret_cast<float*>(&v_lds0[0][0]) + wave * 128;
    if (pair == 1) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(xs + ((cb * 4 + r4) * 64 + L) * 4) =
              make_float4(st.acc[cb][r4 * 4], st.acc[cb][r4 * 4 + 1], st.acc[cb][r4 * 4 + 2], st.acc[cb][r4 * 4 + 3]);
      ms[L] = st.m;
      ms[64 + L] = st.den;
    }
    __syncthreads();
    if (pair == 1) return;
    // pair 0: the two running states on the common maximum (acc and den alike)
    const float m1 = ms[L], den1 = ms[64 + L];
    const float mn = fmaxf(st.m, m1);
    const float f0 = texp2(st.m - mn), f1 = texp2(m1 - mn);
    st.den = __builtin_fmaf(den1, f1, st.den * f0);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float4 x = *reinterpret_cast<const float4*>(xs + ((cb * 4 + r4) * 64 + L) * 4);
        const float xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) st.acc[cb][r4 * 4 + i] = __builtin_fmaf(xv[i], f1, st.acc[cb][r4 * 4 + i] * f0);
      }
    st.m = mn;
  }

  // ---- epilogue: out = fma(acc / den, scale, mean) (prefill_sm80.cu:466-487)
  if (!row_ok) return;
  const float inv = st.den > 0.f ? 1.f / st.den : 0.f;
  const int64_t obase = b * a.osb + qh * a.osh + (int64_t)qrow * a.ost;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int ch = cb * 32 + 8 * r4 + 4 * half;
      const float4 mean = *reinterpret_cast<const float4*>(vms_lds + ch);
      const float4 scale = *reinterpret_cast<const float4*>(vms_lds + D + ch);
      const float mv[4] = {mean.x, mean.y, mean.z, mean.w}, sv[4] = {scale.x, scale.y, scale.z, scale.w};
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = __builtin_fmaf(st.acc[cb][r4 * 4 + i] * inv, sv[i], mv[i]);
      if (a.out_dtype == 0) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase + ch) = make_float4(v[0], v[1], v[2], v[3]);
      } else if (a.out_dtype == 1) {
        const uint32_t lo = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
        const uint32_t hi = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase + ch) = make_uint2(lo, hi);
      } else {
        const uint32_t lo = f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16);
        const uint32_t hi = f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase + ch) = make_uint2(lo, hi);
      }
    }
}

}  // namespace tri
