// Rotate + quantize kernels for gfx950: Q per-token INT8/INT4 codes, per-channel
// K/V statistics, centred+rotated K records with per-(tile, 16-key group) scales,
// and the normalised V records.  All arithmetic is IEEE fp32 with the
// reference's operation order, so codes and scales are bit-exact.
//
// Reference semantics: triattention/kernels/cuda/common_device.cuh:1-172.
#include "common.h"

namespace tri {

// One 128-feature row per 8 lanes (16 features per lane, rotated with DPP lane
// moves by rotate128_x16), 32 rows per 256-thread block.
// common_device.cuh:1-28 (quantize_q_kernel).
__global__ __launch_bounds__(256) void quantize_q_kernel(const uint16_t* __restrict__ q, int64_t sb, int64_t sh,
                                                         int64_t st, int hq, int t, int8_t* __restrict__ q8,
                                                         float* __restrict__ qa, uint8_t* __restrict__ q4,
                                                         float* __restrict__ qa4) {
  const int sub = threadIdx.x & 7, row = blockIdx.x * 32 + (threadIdx.x >> 3), h = blockIdx.y, b = blockIdx.z;
  if (row >= t) return;  // whole 8-lane groups leave together
  const uint16_t* src = q + b * sb + h * sh + (int64_t)row * st + sub * 16;
  float x[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint2 raw = *reinterpret_cast<const uint2*>(src + 4 * i);
    x[4 * i] = bf16f(raw.x & 0xffffu);
    x[4 * i + 1] = bf16f(raw.x >> 16);
    x[4 * i + 2] = bf16f(raw.y & 0xffffu);
    x[4 * i + 3] = bf16f(raw.y >> 16);
  }
  rotate128_x16(x, sub);
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(x[i]));
  m = lanes8_max(m);
  const int64_t r = ((int64_t)b * hq + h) * t + row;
  const float inv = m > 0.f ? 127.f / m : 0.f;
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    w[k] = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[k] |= ((uint32_t)(int)__builtin_rintf(x[4 * k + i] * inv) & 0xffu) << (8 * i);
  }
  *reinterpret_cast<uint4*>(q8 + r * D + sub * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  if (sub == 0) qa[r] = m / 127.f;
  if (q4 != nullptr) {
    const float inv4 = m > 0.f ? 7.f / m : 0.f;
    uint32_t nib[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) nib[i >> 3] |= ((uint32_t)(int)__builtin_rintf(x[i] * inv4) & 0xfu) << (4 * (i & 7));
    uint32_t* dst = reinterpret_cast<uint32_t*>(q4 + r * (D / 2) + sub * 8);
    dst[0] = nib[0];
    dst[1] = nib[1];
    if (sub == 0) qa4[r] = m / 7.f;
  }
}

// Per channel: sequential sum/max/min over tokens t = blk, blk+64, ...
// common_device.cuh:32-42 (partial_kernel).  partial [B][H][64][3][128].
// Lane i takes channels 2i and 2i + 1 (one 4-byte load per token; rows are 8-byte aligned) and
// issues the loads of STAT_DEPTH tokens before it adds them, in token order, so each channel's
// sum is formed in the reference's order while 32 loads per lane are in flight (C2's K: 14 us
// against 22 us with 2-byte loads four deep; 64 deep, or 8 channels per lane with two rows per
// load, measured no faster).
constexpr int STAT_DEPTH = 32;
__global__ __launch_bounds__(64) void partial_kernel(const uint16_t* __restrict__ x, int64_t sb, int64_t sh,
                                                     int64_t st, int h, int t, float* __restrict__ partial) {
  const int blk = blockIdx.x, hd = blockIdx.y, b = blockIdx.z, c = 2 * threadIdx.x;
  const uint16_t* base = x + b * sb + hd * sh + c;
  float sum0 = 0.f, sum1 = 0.f, hi0 = -3.402823466e38f, hi1 = hi0, lo0 = 3.402823466e38f, lo1 = lo0;
  for (int tk = blk; tk < t; tk += STAT_DEPTH * STAT_BLOCKS) {
    uint32_t w[STAT_DEPTH];
#pragma unroll
    for (int j = 0; j < STAT_DEPTH; ++j)
      if (tk + j * STAT_BLOCKS < t) w[j] = *reinterpret_cast<const uint32_t*>(base + (int64_t)(tk + j * STAT_BLOCKS) * st);
#pragma unroll
    for (int j = 0; j < STAT_DEPTH; ++j)
      if (tk + j * STAT_BLOCKS < t) {
        const float v0 = bf16f((uint16_t)(w[j] & 0xffffu)), v1 = bf16f((uint16_t)(w[j] >> 16));
        sum0 += v0;
        sum1 += v1;
        hi0 = fmaxf(hi0, v0);
        hi1 = fmaxf(hi1, v1);
        lo0 = fminf(lo0, v0);
        lo1 = fminf(lo1, v1);
      }
  }
  float* o = partial + ((((int64_t)b * h + hd) * STAT_BLOCKS + blk) * 3) * D + c;
  *reinterpret_cast<float2*>(o) = make_float2(sum0, sum1);
  *reinterpret_cast<float2*>(o + D) = make_float2(hi0, hi1);
  *reinterpret_cast<float2*>(o + 2 * D) = make_float2(lo0, lo1);
}

// mean = (sum of block sums in block order) / T, scale = range/127 (1 if 0),
// inv = 1/scale; identity mode writes (0, 1, 1).  common_device.cuh:44-56.
__global__ __launch_bounds__(128) void finalize_kernel(const float* __restrict__ partial, float* __restrict__ stat,
                                                       int h, int t, int identity) {
  const int hd = blockIdx.x, b = blockIdx.y, c = threadIdx.x;
  const int64_t hb = (int64_t)b * h + hd;
  float mean = 0.f, scale = 1.f;
  if (!identity) {
    const float* in = partial + hb * STAT_BLOCKS * 3 * D + c;
    float sum = 0.f, hi = -3.402823466e38f, lo = 3.402823466e38f;
    // (unrolled: the 192 loads issue together, and the sum still runs in block order)
#pragma unroll
    for (int blk = 0; blk < STAT_BLOCKS; ++blk) {
      sum += in[blk * 3 * D];
      hi = fmaxf(hi, in[blk * 3 * D + D]);
      lo = fminf(lo, in[blk * 3 * D + 2 * D]);
    }
    mean = sum / (float)t;
    const float range = fmaxf(hi - mean, mean - lo);
    scale = range > 0.f ? range / 127.f : 1.f;
  }
  stat[hb * 3 * D + c] = mean;
  stat[hb * 3 * D + D + c] = scale;
  stat[hb * 3 * D + 2 * D + c] = 1.f / scale;
}

// y = R(k - mean) of one 64-key tile: rows src + r * st for r < rows (zeros past); the INT8 record rec8
// with its four group scales ka, and the INT4 record rec4 with ka4 (either pair may be null).  Wave w
// owns the 16-key group w, one key per 8 lanes (16 features per lane, DPP rotation), two passes of 8
// keys; c8 / c4 are the workgroup's LDS staging.  256 threads.
// common_device.cuh:58-131 (quantize_k_kernel).
// Extension: rec4x (with rec4; may be null) receives the INT4 codes once more, expanded to one byte of
// 16 * code each in the INT8 record's layout (8 KiB): the bytes the prefill kernel would otherwise expand
// from rec4 in every tile it reads.
__device__ __forceinline__ void quantize_k_tile(const uint16_t* __restrict__ src, int64_t st, int rows,
                                                const float* __restrict__ mean, uint8_t* __restrict__ rec8,
                                                float* __restrict__ ka, uint8_t* __restrict__ rec4,
                                                float* __restrict__ ka4, uint8_t (*c8)[D], uint8_t (*c4)[D],
                                                uint8_t* __restrict__ rec4x = nullptr) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, sub = lane & 7;
  float mc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) mc[i] = mean[sub * 16 + i];
  float y[2][16];
  float cm = 0.f;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int r = wave * 16 + it * 8 + (lane >> 3);
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = 0.f;
    if (r < rows) {
      const uint16_t* row = src + (int64_t)r * st + sub * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 raw = *reinterpret_cast<const uint2*>(row + 4 * i);
        x[4 * i] = bf16f(raw.x & 0xffffu) - mc[4 * i];
        x[4 * i + 1] = bf16f(raw.x >> 16) - mc[4 * i + 1];
        x[4 * i + 2] = bf16f(raw.y & 0xffffu) - mc[4 * i + 2];
        x[4 * i + 3] = bf16f(raw.y >> 16) - mc[4 * i + 3];
      }
    }
    rotate128_x16(x, sub);  // every lane of the wave takes part (padded rows rotate zeros)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      y[it][i] = x[i];
      cm = fmaxf(cm, fabsf(x[i]));
    }
  }
  cm = wave_max(cm);
  const float inv = cm > 0.f ? 127.f / cm : 0.f, inv4 = cm > 0.f ? 7.f / cm : 0.f;
  if (lane == 0) {
    if (rec8 != nullptr) ka[wave] = cm > 0.f ? cm / 127.f : 1.f;
    if (rec4 != nullptr) ka4[wave] = cm > 0.f ? cm / 7.f : 1.f;
  }
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int r = wave * 16 + it * 8 + (lane >> 3);
    uint32_t w8[4], w4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      w8[q] = 0u;
      w4[q] = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w8[q] |= ((uint32_t)(int)__builtin_rintf(y[it][4 * q + i] * inv) & 0xffu) << (8 * i);
        w4[q] |= ((uint32_t)(int)__builtin_rintf(y[it][4 * q + i] * inv4) & 0xfu) << (8 * i);
      }
    }
    *reinterpret_cast<uint4*>(&c8[r][sub * 16]) = make_uint4(w8[0], w8[1], w8[2], w8[3]);
    *reinterpret_cast<uint4*>(&c4[r][sub * 16]) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
  __syncthreads();
  if (rec8 != nullptr) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int s = tid + it * 256, F = s >> 6, L = s & 63, kb = F >> 2, ks = F & 3;
      const int key = kb * 32 + (L & 31), f0 = ks * 32 + 16 * (L >> 5);
      *reinterpret_cast<uint4*>(rec8 + F * 1024 + L * 16) = *reinterpret_cast<const uint4*>(&c8[key][f0]);
    }
  }
  if (rec4 == nullptr) return;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int s = tid + it * 256, F = s >> 6, L = s & 63, kb = F >> 2, ks = F & 3;
    const int key = kb * 32 + (L & 31), f0 = ks * 32 + 16 * (L >> 5);
    const uint4 n = *reinterpret_cast<const uint4*>(&c4[key][f0]);  // one nibble value per byte
    const uint32_t w0 = n.x | (n.y << 4), w1 = n.z | (n.w << 4);
    *reinterpret_cast<uint2*>(rec4 + (F >> 1) * 1024 + L * 16 + (F & 1) * 8) = make_uint2(w0, w1);
    if (rec4x != nullptr)
      *reinterpret_cast<uint4*>(rec4x + F * 1024 + L * 16) =
          make_uint4((n.x << 4) & 0xf0f0f0f0u, (n.y << 4) & 0xf0f0f0f0u, (n.z << 4) & 0xf0f0f0f0u,
                     (n.w << 4) & 0xf0f0f0f0u);
  }
}

// quantize_k_tile for every (tile, KV head, sequence): K [B][Hk][T][128] into [B][Hk][tiles] records.
__global__ __launch_bounds__(256) void quantize_k_kernel(const uint16_t* __restrict__ k, int64_t sb, int64_t sh,
                                                         int64_t st, const float* __restrict__ kstat, int hk, int t,
                                                         uint8_t* __restrict__ k8, float* __restrict__ ka,
                                                         uint8_t* __restrict__ k4, float* __restrict__ ka4,
                                                         uint8_t* __restrict__ k4x) {
  __shared__ __align__(16) uint8_t c8[BN][D];
  __shared__ __align__(16) uint8_t c4[BN][D];
  const int tile = blockIdx.x, hd = blockIdx.y, b = blockIdx.z, tiles = (t + BN - 1) / BN;
  const int64_t hb = (int64_t)b * hk + hd, rec = hb * tiles + tile;
  quantize_k_tile(k + b * sb + hd * sh + (int64_t)tile * BN * st, st, t - tile * BN, kstat + hb * 3 * D,
                  k8 + rec * K8_BYTES, ka + rec * 4, k4 != nullptr ? k4 + rec * K4_BYTES : nullptr,
                  k4 != nullptr ? ka4 + rec * 4 : nullptr, c8, c4, k4x != nullptr ? k4x + rec * K8_BYTES : nullptr);
}

// v' = (v - mean) * inv of one 64-key tile (rows src + r * st for r < rows, zeros past) into the V16
// (fp16), V8 and V4 records (any may be null); vn is the workgroup's LDS staging.  256 threads.
// common_device.cuh:132-172 (vnorm, pack_v_kernel).
// Extension: v8s (with v8; may be null) receives -127 times each channel's sum of the tile's 64 V8 codes
// (int32 [128], channel order), the value the prefill's P V product starts from (vsum: LDS of 128 ints).
__device__ __forceinline__ void pack_v_tile(const uint16_t* __restrict__ src, int64_t st, int rows,
                                            const float* __restrict__ mean, const float* __restrict__ inv,
                                            uint8_t* __restrict__ v16, uint8_t* __restrict__ v8,
                                            uint8_t* __restrict__ v4, float (*vn)[D + 1],
                                            int32_t* __restrict__ v8s = nullptr, int* vsum = nullptr) {
  const int tid = threadIdx.x;
  if (v8s != nullptr && tid < D) vsum[tid] = 0;
  for (int i = tid; i < BN * D / 4; i += 256) {
    const int r = i / (D / 4), c0 = (i % (D / 4)) * 4;
    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (r < rows) {
      const uint2 raw = *reinterpret_cast<const uint2*>(src + (int64_t)r * st + c0);
      x[0] = (bf16f(raw.x & 0xffffu) - mean[c0]) * inv[c0];
      x[1] = (bf16f(raw.x >> 16) - mean[c0 + 1]) * inv[c0 + 1];
      x[2] = (bf16f(raw.y & 0xffffu) - mean[c0 + 2]) * inv[c0 + 2];
      x[3] = (bf16f(raw.y >> 16) - mean[c0 + 3]) * inv[c0 + 3];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) vn[r][c0 + j] = x[j];
  }
  __syncthreads();
  if (v16 != nullptr) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int s = tid + it * 256, F = s >> 6, L = s & 63, kh = F & 1, kb = (F >> 1) & 1, cb = F >> 2;
      const int ch = cb * 32 + (L & 31), g = L >> 5;
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int k0 = kb * 32 + 8 * (2 * kh + e / 4) + 4 * g + e % 4;
        w[e / 2] = (uint32_t)f32_to_f16_bits(vn[k0][ch]) | ((uint32_t)f32_to_f16_bits(vn[k0 + 1][ch]) << 16);
      }
      *reinterpret_cast<uint4*>(v16 + F * 1024 + L * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  if (v8 == nullptr && v4 == nullptr) return;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int s = tid + it * 256, F = s >> 6, L = s & 63, kb = F & 1, cb = F >> 1;
    const int ch = cb * 32 + (L & 31), g = L >> 5;
    uint32_t b8[4] = {0, 0, 0, 0}, b4[4] = {0, 0, 0, 0};
    int sum8 = 0;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const float x = vn[kb * 32 + 8 * (p / 4) + 4 * g + p % 4][ch];
      const int q8 = max(-127, min(127, (int)__builtin_rintf(x)));
      const int q4 = max(-7, min(7, (int)__builtin_rintf(x * (7.f / 127.f))));
      b8[p / 4] |= ((uint32_t)q8 & 0xffu) << (8 * (p % 4));
      b4[p / 4] |= ((uint32_t)q4 & 0xfu) << (8 * (p % 4));
      sum8 += q8;
    }
    // four threads hold 16 keys each of channel ch: integer adds, so the sum is order-free
    if (v8s != nullptr) atomicAdd(&vsum[ch], sum8);
    if (v8 != nullptr) *reinterpret_cast<uint4*>(v8 + F * 1024 + L * 16) = make_uint4(b8[0], b8[1], b8[2], b8[3]);
    if (v4 != nullptr)
      *reinterpret_cast<uint2*>(v4 + (F >> 1) * 1024 + L * 16 + (F & 1) * 8) =
          make_uint2(b4[0] | (b4[1] << 4), b4[2] | (b4[3] << 4));
  }
  if (v8s != nullptr) {
    __syncthreads();
    if (tid < D) v8s[tid] = -127 * vsum[tid];
  }
}

// pack_v_tile for every (tile, KV head, sequence): V [B][Hk][T][128] into [B][Hk][tiles] records.
__global__ __launch_bounds__(256) void pack_v_kernel(const uint16_t* __restrict__ v, int64_t sb, int64_t sh,
                                                     int64_t st, const float* __restrict__ vstat, int hk, int t,
                                                     uint8_t* __restrict__ v16, uint8_t* __restrict__ v8,
                                                     uint8_t* __restrict__ v4, int32_t* __restrict__ v8s) {
  __shared__ float vn[BN][D + 1];
  __shared__ int vsum[D];
  const int tile = blockIdx.x, hd = blockIdx.y, b = blockIdx.z, tiles = (t + BN - 1) / BN;
  const int64_t hb = (int64_t)b * hk + hd, rec = hb * tiles + tile;
  const float* mean = vstat + hb * 3 * D;
  pack_v_tile(v + b * sb + hd * sh + (int64_t)tile * BN * st, st, t - tile * BN, mean, mean + 2 * D,
              v16 != nullptr ? v16 + rec * V16_BYTES : nullptr, v8 != nullptr ? v8 + rec * V8_BYTES : nullptr,
              v4 != nullptr ? v4 + rec * V4_BYTES : nullptr, vn, v8s != nullptr ? v8s + rec * D : nullptr, vsum);
}

}  // namespace tri
