// Split-KV decode over the quantized cache, plus the merge with the bf16 tail.
//
// Reference semantics: triattention/kernels/cuda/common_device.cuh:178-469
// (decode_tile, decode_kernel, decode_merge_kernel) and the cache metadata of
// triattention/kernels/decode.py:24-67.
//
// One 64-lane wave per (sequence, KV head, split).  The kept tiles of a split
// stream straight from HBM into MFMA operand registers (one 16-byte load per
// lane per 1 KiB fragment, next tile prefetched while the current one is
// processed); no LDS staging is needed because every fragment is consumed by
// exactly one wave.  The g <= 8 query heads of the KV group occupy columns
// 0..g-1 of the 32-wide MFMA B operand.
#include "common.h"

namespace tri {

struct DecodeArgs {
  const uint16_t* q;        // [B][Hq][1][128] bf16, strides qsb, qsh
  const uint8_t* k8c;       // compacted K8 records
  const uint8_t* k4c;       // compacted K4 records (may be null)
  const float* ka;          // [B][Hk][tiles_max][4]
  const float* ka4;         // [B][Hk][tiles_max][4] (may be null)
  const int32_t* entry;     // [B][Hk][maxn] tile index
  const int32_t* kinfo;     // rowmask | is4 << 8 | kslot << 9
  const int32_t* count;     // [B][Hk]
  const int32_t* fmt;       // [B][tiles_max]: 1 = INT8 V, 2 = INT4 V
  const int32_t* slot;      // [B][Hk][maxn] V record slot
  const uint8_t* v8c;
  const uint8_t* v4c;
  const int32_t* prompt;    // [B]
  float* pm;                // [B][Hq][splits]
  float* pl;
  float* po;                // [B][Hq][splits][128]
  int64_t qsb, qsh;
  int hq, hk, maxn, per, tiles_max, splits;
  float sm_log2;
};

__device__ __forceinline__ float dx32_max(float v) { return fmaxf(v, __shfl_xor(v, 32, 64)); }

__global__ __launch_bounds__(64) void decode_kernel(DecodeArgs a) {
  __shared__ __align__(16) int8_t q8s[MAX_GROUP][D];
  __shared__ __align__(16) int8_t q4s[MAX_GROUP][D];
  __shared__ float qsc[MAX_GROUP], qsc4[MAX_GROUP];
  const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int L = threadIdx.x, lq = L & 31, half = L >> 5;
  const int g = a.hq / a.hk;
  const int prompt = a.prompt[b];
  const int64_t hb = (int64_t)b * a.hk + kh;
  const int cnt = a.count[hb], first = split * a.per, last = min(cnt, first + a.per);

  // ---- in-kernel Q quantization of the g rows (common_device.cuh:291-315)
#pragma unroll
  for (int it = 0; it < MAX_GROUP / 2; ++it) {
    const int r = it * 2 + half;
    float xv[4] = {0.f, 0.f, 0.f, 0.f};
    if (r < g) {
      const uint2 raw = *reinterpret_cast<const uint2*>(a.q + b * a.qsb + (int64_t)(kh * g + r) * a.qsh + lq * 4);
      xv[0] = bf16f(raw.x & 0xffffu); xv[1] = bf16f(raw.x >> 16);
      xv[2] = bf16f(raw.y & 0xffffu); xv[3] = bf16f(raw.y >> 16);
    }
    rotate128_x4(xv, lq);
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fabsf(xv[i]));
    mx = warp32_max(mx);
    const float inv = mx > 0.f ? 127.f / mx : 0.f, inv4 = mx > 0.f ? 7.f / mx : 0.f;
    uint32_t w8 = 0, w4 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w8 |= ((uint32_t)(int)__builtin_rintf(xv[i] * inv) & 0xffu) << (8 * i);
      const int c4 = (((int)__builtin_rintf(xv[i] * inv4) & 0xf) ^ 8) - 8;
      w4 |= ((uint32_t)c4 & 0xffu) << (8 * i);
    }
    *reinterpret_cast<uint32_t*>(&q8s[r][lq * 4]) = r < g ? w8 : 0u;
    *reinterpret_cast<uint32_t*>(&q4s[r][lq * 4]) = r < g ? w4 : 0u;
    if (lq == 0) {
      qsc[r] = (r < g && mx > 0.f) ? mx / 127.f * a.sm_log2 : 1.17549435e-38f;
      qsc4[r] = (r < g && mx > 0.f) ? mx / 7.f * a.sm_log2 : 1.17549435e-38f;
    }
  }
  __syncthreads();
  v4i qf8[4], qf4[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    v4i z = {0, 0, 0, 0};
    qf8[ks] = lq < g ? *reinterpret_cast<const v4i*>(&q8s[lq][ks * 32 + 16 * half]) : z;
    qf4[ks] = lq < g ? *reinterpret_cast<const v4i*>(&q4s[lq][ks * 32 + 16 * half]) : z;
  }
  const float qs8 = lq < g ? qsc[lq] : 1.17549435e-38f, qs4 = lq < g ? qsc4[lq] : 1.17549435e-38f;

  v16f acc[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[cb][r] = 0.f;
  float m = -3.402823466e38f, den = 0.f;
  const int64_t mbase = hb * a.maxn;

  for (int e = first; e < last; ++e) {
    const int j = a.entry[mbase + e], info = a.kinfo[mbase + e];
    const int is4 = (info >> 8) & 1, kslot = (int)((unsigned)info >> 9);
    const unsigned rowmask = info & 0xff;
    const int vs = a.slot[mbase + e], vf = a.fmt[(int64_t)b * a.tiles_max + j];
    // ---- K fragments
    v4i kf[8];
    if (is4) {
      const uint8_t* src = a.k4c + (int64_t)kslot * K4_BYTES + L * 8;
#pragma unroll
      for (int F = 0; F < 8; ++F) {
        const uint2 w = *reinterpret_cast<const uint2*>(src + F * 512);
        kf[F] = v4i{(int)nib_lo16(w.x), (int)nib_hi16(w.x), (int)nib_lo16(w.y), (int)nib_hi16(w.y)};
      }
    } else {
      const uint8_t* src = a.k8c + (int64_t)kslot * K8_BYTES + L * 16;
#pragma unroll
      for (int F = 0; F < 8; ++F) kf[F] = *reinterpret_cast<const v4i*>(src + F * 1024);
    }
    // ---- V fragments (V4 unpacked to 16*code)
    v4i vfr[8];
    if (vf == 1) {
      const uint8_t* src = a.v8c + (int64_t)vs * V8_BYTES + L * 16;
#pragma unroll
      for (int F = 0; F < 8; ++F) vfr[F] = *reinterpret_cast<const v4i*>(src + F * 1024);
    } else {
      const uint8_t* src = a.v4c + (int64_t)vs * V4_BYTES + L * 8;
#pragma unroll
      for (int F = 0; F < 8; ++F) {
        const uint2 w = *reinterpret_cast<const uint2*>(src + F * 512);
        vfr[F] = v4i{(int)nib_lo16(w.x), (int)nib_hi16(w.x), (int)nib_lo16(w.y), (int)nib_hi16(w.y)};
      }
    }
    // ---- S^T
    v16i s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) s[kb] = mfma_i8(kf[kb * 4 + ks], is4 ? qf4[ks] : qf8[ks], s[kb]);
    const bool row_on = lq < g && ((rowmask >> lq) & 1u);
    const float qs = is4 ? qs4 : qs8;
    const float* kt = (is4 ? a.ka4 : a.ka) + (hb * a.tiles_max + j) * 4;
    float slope[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) slope[gi] = qs * kt[gi];
    const float slope1 = qs * fmaxf(fmaxf(kt[0], kt[1]), fmaxf(kt[2], kt[3]));
    int dot[2][16];
    bool ok[2][16];
    float tile = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hg = 0; hg < 2; ++hg) {
        bool have = false;
        int mx = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = hg * 8 + i;
          const int key = j * BN + kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          const int d = is4 ? (s[kb][r] >> 4) : s[kb][r];
          dot[kb][r] = d;
          ok[kb][r] = row_on && key < prompt;
          if (ok[kb][r] && (!have || d > mx)) { mx = d; have = true; }
        }
        if (have) tile = fmaxf(tile, slope[kb * 2 + hg] * (float)mx);
      }
    tile = dx32_max(tile);
    const float n = fmaxf(m, tile), alpha = texp2(m - n);
    m = n;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cb][r] *= alpha;
    }
    const float levels = vf == 1 ? 255.f : 15.f;
    const bool any = tile > -__builtin_inff();
    float base = any ? tile : n;
    base += __builtin_fmaf(slope1, 0.75f, fabsf(base) * 2.4e-7f);
    const float bq = any ? texp2(base - n) / levels : 0.f;
    const float restore = vf == 1 ? bq : bq * (127.f / 7.f);
    float c[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) c[gi] = is4 ? -base : (-slope[gi] * MAGIC) - base;
    uint32_t pw[2][4];
    uint32_t rs = 0;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        uint32_t y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = qd * 4 + i, gi = kb * 2 + (r >> 3);
          const int d = dot[kb][r];
          float arg;
          uint32_t dith;
          if (ok[kb][r]) {
            const float xm = __uint_as_float(MAGIC_BITS + (uint32_t)d);
            arg = is4 ? __builtin_fmaf(slope[gi], (float)d, c[gi]) : __builtin_fmaf(slope[gi], xm, c[gi]);
            dith = ((uint32_t)d & 0xffu) | 0x47400000u;
          } else {
            arg = -__builtin_inff();
            dith = 0x47400000u;
          }
          y[i] = __float_as_uint(__builtin_fmaf(texp2(arg), levels, __uint_as_float(dith)));
        }
        const uint32_t w = pack_byte1(y[0], y[1], y[2], y[3]);
        rs = __builtin_amdgcn_udot4(w, 0x01010101u, rs, false);
        pw[kb][qd] = vf == 1 ? (w ^ 0x7f7f7f7fu) : w;
      }
    rs += __shfl_xor(rs, 32, 64);
    den = __builtin_fmaf((float)rs, bq, den * alpha);
    const v4i b0 = {(int)pw[0][0], (int)pw[0][1], (int)pw[0][2], (int)pw[0][3]};
    const v4i b1 = {(int)pw[1][0], (int)pw[1][1], (int)pw[1][2], (int)pw[1][3]};
    if (vf == 1) {
      const v4i neg127 = {(int)0x81818181u, (int)0x81818181u, (int)0x81818181u, (int)0x81818181u};
      const float nr = -restore;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        v16i d = {};
        d = mfma_i8(vfr[cb * 2], neg127, d);
        d = mfma_i8(vfr[cb * 2 + 1], neg127, d);
        d = mfma_i8(vfr[cb * 2], b0, d);
        d = mfma_i8(vfr[cb * 2 + 1], b1, d);  // = -sum P v
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cb][r] = __builtin_fmaf((float)d[r], nr, acc[cb][r]);
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        v16i d = {};
        d = mfma_i8(vfr[cb * 2], b0, d);
        d = mfma_i8(vfr[cb * 2 + 1], b1, d);  // = 16 * sum P v
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cb][r] = __builtin_fmaf((float)(d[r] >> 4), restore, acc[cb][r]);
      }
    }
  }
  // ---- split partials (common_device.cuh:355-370)
  if (lq < g) {
    const int64_t idx = ((int64_t)b * a.hq + kh * g + lq) * a.splits + split;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int ch = cb * 32 + 8 * r4 + 4 * half;
        *reinterpret_cast<float4*>(a.po + idx * D + ch) =
            make_float4(acc[cb][r4 * 4], acc[cb][r4 * 4 + 1], acc[cb][r4 * 4 + 2], acc[cb][r4 * 4 + 3]);
      }
    if (half == 0) {
      a.pm[idx] = m;
      a.pl[idx] = den;
    }
  }
}

struct MergeArgs {
  const float* pm;
  const float* pl;
  const float* po;
  const float* vstat;   // [B][Hk][3][128]
  const float* kstat;
  const uint16_t* q;
  uint16_t* ktail;      // [B][Hk][max_tail][128], strides tsb, tsh, tst
  uint16_t* vtail;
  const uint16_t* kcur;  // [B][Hk][1][128], strides csb, csh
  const uint16_t* vcur;
  const int64_t* step;
  void* out;             // [B][Hq][1][128], strides osb, osh
  int out_dtype;         // 0 = fp32, 1 = bf16
  int64_t qsb, qsh, tsb, tsh, tst, csb, csh, osb, osh;
  int hq, hk, splits, max_tail;
  float sm_log2;
};

constexpr int MAX_TAIL = 1024;

// LSE merge of the split partials with the exact bf16 tail
// (common_device.cuh:373-469).  One 256-thread workgroup per (sequence, q-head).
__global__ __launch_bounds__(256) void decode_merge_kernel(MergeArgs a) {
  __shared__ float ts[MAX_TAIL];
  __shared__ float wmax[8], wl[4];
  __shared__ float wo[4][D];
  const int hq = blockIdx.x, b = blockIdx.y, g = a.hq / a.hk, kh = hq / g;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, sub = lane >> 5;
  const int prior = (int)min((int64_t)a.max_tail - 1, *a.step), tail = prior + 1;
  const int64_t hb = (int64_t)b * a.hk + kh;
  const float* vmean = a.vstat + hb * 3 * D;
  const float* vscale = vmean + D;
  const uint16_t* kc = a.kcur + b * a.csb + kh * a.csh;
  const uint16_t* vc = a.vcur + b * a.csb + kh * a.csh;
  if (hq % g == 0 && tid < D) {
    a.ktail[b * a.tsb + kh * a.tsh + prior * a.tst + tid] = kc[tid];
    a.vtail[b * a.tsb + kh * a.tsh + prior * a.tst + tid] = vc[tid];
  }
  // tail scores: 32-lane fma chains over 4 channels each, then a xor butterfly
  float qv[4], kmu[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qv[i] = bf16f(a.q[b * a.qsb + hq * a.qsh + l32 * 4 + i]);
    kmu[i] = a.kstat[hb * 3 * D + l32 * 4 + i];
  }
  for (int t = wave * 2 + sub; t < tail; t += 8) {
    const uint16_t* kv = t < prior ? a.ktail + b * a.tsb + kh * a.tsh + (int64_t)t * a.tst : kc;
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) part = __builtin_fmaf(qv[i], bf16f(kv[l32 * 4 + i]) - kmu[i], part);
#pragma unroll
    for (int o = 16; o; o >>= 1) part += __shfl_xor(part, o, 32);
    if (l32 == 0) ts[t] = part * a.sm_log2;
  }
  __syncthreads();
  const int64_t pbase = ((int64_t)b * a.hq + hq) * a.splits;
  float m = -3.402823466e38f;
  for (int s = tid; s < a.splits; s += 256) m = fmaxf(m, a.pm[pbase + s]);
  for (int t = tid; t < tail; t += 256) m = fmaxf(m, ts[t]);
#pragma unroll
  for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) wmax[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  // four interleaved split accumulators, summed in order
  float l = 0.f, o0 = 0.f, o1 = 0.f;
  for (int s = wave; s < a.splits; s += 4) {
    const float w = texp2(a.pm[pbase + s] - m);
    l = __builtin_fmaf(a.pl[pbase + s], w, l);
    const float2 p = *reinterpret_cast<const float2*>(a.po + (pbase + s) * D + lane * 2);
    o0 = __builtin_fmaf(p.x, w, o0);
    o1 = __builtin_fmaf(p.y, w, o1);
  }
  if (lane == 0) wl[wave] = l;
  wo[wave][lane * 2] = o0;
  wo[wave][lane * 2 + 1] = o1;
  __syncthreads();
  if (tid >= D) return;
  float total = 0.f, acc = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    total += wl[w];
    acc += wo[w][tid];
  }
  acc = __builtin_fmaf(acc, vscale[tid], total * vmean[tid]);
  const uint16_t* vt = a.vtail + b * a.tsb + kh * a.tsh + tid;
  for (int t = 0; t < prior; ++t) {
    const float e = texp2(ts[t] - m);
    total += e;
    acc = __builtin_fmaf(e, bf16f(vt[(int64_t)t * a.tst]), acc);
  }
  const float e = texp2(ts[prior] - m);
  total += e;
  acc = __builtin_fmaf(e, bf16f(vc[tid]), acc);
  const float r = acc / total;
  if (a.out_dtype == 0) static_cast<float*>(a.out)[b * a.osb + hq * a.osh + tid] = r;
  else static_cast<uint16_t*>(a.out)[b * a.osb + hq * a.osh + tid] = f32_to_bf16(r);
}

}  // namespace tri
