// Streaming-read probe: the HBM read rate a kernel with no compute reaches on this device, for a
// given byte count and launch shape.  It is the practical ceiling the split-KV decode kernel's
// record stream is compared against (the decode kernel reads each record once, in 1 KiB
// fragments of 16 bytes per lane, as this probe does).  No reference counterpart.
#include "common.h"

namespace tri {

constexpr int PROBE_RECORD = 8192;  // bytes per record (a K8 / V8 record)

// Wave i reads records [i * per, (i + 1) * per) in order, DEPTH records in flight: eight 16-byte
// non-temporal loads per lane per record (the decode kernel's cache policy), through a descriptor per record (loads past the array read zeros
// without touching memory).  The XOR of everything read goes to sink[0] only if it equals a value
// no real input produces, so the loads cannot be dropped and nothing is written in practice.
template <int DEPTH>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* base, int64_t records, int per,
                                                          int32_t* sink) {
  const int L = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t r0 = wave * per, r1 = min(records, r0 + per);
  v4i acc = {0, 0, 0, 0};
  v4i buf[DEPTH][8];
  auto load = [&](int d, int64_t r) {
    const bool ok = r < r1;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(base + (ok ? r : 0) * PROBE_RECORD), (short)0, ok ? PROBE_RECORD : 0, 0x00020000);
#pragma unroll
    for (int f = 0; f < 8; ++f) buf[d][f] = __builtin_amdgcn_raw_buffer_load_b128(rs, L * 16 + f * 1024, 0, LOAD_STREAM);
  };
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load(d, r0 + d);
  for (int64_t r = r0; r < r1; r += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
#pragma unroll
      for (int f = 0; f < 8; ++f) acc ^= buf[d][f];
      load(d, r + d + DEPTH);
    }
  }
  const int x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x5a17c0de) sink[0] = x;
}

}  // namespace tri

namespace tri {

// Issue-cost probe: how many SIMD cycles the instruction kinds of the attention tiles take when one
// or more waves issue them.  One workgroup per CU of 256 * W threads (W waves per SIMD: wave i runs
// on SIMD i % 4; 100 KiB of LDS keeps every other workgroup off the CU), each wave timing ITERS
// iterations of MODE with s_memtime (shader clock) and s_memrealtime (100 MHz), written to
// out[2 * wave], out[2 * wave + 1].  Modes (per iteration):
//   0: 32 independent v_fma_f32            1: 8 independent v_exp_f32
//   2: 24 v_fma_f32 and 8 v_exp_f32       3: 4 independent v_mfma_i32_32x32x32_i8
//   4: 4 independent v_mfma_f32_32x32x16_bf16
//   5: 4 v_mfma_i32_32x32x32_i8 and 64 v_fma_f32 in the same wave
//   6: the first wave of each SIMD 4 v_mfma_i32_32x32x32_i8, the others 32 v_fma_f32
// and, per wave, 4 v_mfma_i32_32x32x32_i8 and 96 v_fma_f32 (the quantized tile's 1 : 24 ratio) as
//   7: spread, each MFMA followed by 24 fma           8: the 4 MFMAs back to back, then the 96 fma
//   9: as 8, then a workgroup barrier                 10: as 9, the first fma reading the last MFMA's
//      result (the tile's score -> softmax dependency, every wave in the same phase)
//  11: as 10 in two halves split by barriers, the odd waves of a SIMD half an iteration behind the even
//      ones (MFMAs of one wave beside the other's fma)
//  12: as 7, then a workgroup barrier
// and, per wave, a tile-shaped iteration: P = 16 v_mfma_i32_32x32x32_i8 interleaved with 128 v_fma_f32,
// S = 200 v_fma_f32 and 32 v_exp_f32 whose first fma reads the last MFMA's result, then a barrier:
//  13: every wave P then S (the waves of a SIMD in the same phase)
//  14: even waves of a SIMD P then S, odd waves S then P (one wave's MFMAs beside the other's S)
// No reference counterpart: a measurement aid for the kernels' cost model.
constexpr int ISSUE_MODES = 15;

__device__ __forceinline__ void probe_fma8(float (&x)[8], float a, float b) {
#pragma unroll
  for (int i = 0; i < 8; ++i) asm volatile("v_fma_f32 %0, %1, %2, %0" : "+v"(x[i]) : "v"(a), "v"(b));
}
__device__ __forceinline__ void probe_exp8(float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) asm volatile("v_exp_f32 %0, %0" : "+v"(x[i]));
}

template <int MODE>
__global__ __launch_bounds__(1024) void issue_probe_kernel(int iters, int64_t* out, float a, float b, int s) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool first_on_simd = wave < 4;
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = a * (float)(lane + i);
  const float fa = x[0] * 0.5f + b, fb = x[1] * 0.25f - a;  // fma operands in registers of their own
  v16i acc[4] = {};
  v16f facc[4] = {};
  const v4i qa = {s, s + 1, s + 2, s + 3}, qb = {s, 2 * s, 3, 4};
  v8bf ba, bb;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ba[i] = (__bf16)(a + (float)i);
    bb[i] = (__bf16)(b - (float)i);
  }
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE == 0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) probe_fma8(x, fa, fb);
    } else if constexpr (MODE == 1) {
      probe_exp8(x);
    } else if constexpr (MODE == 2) {
#pragma unroll
      for (int k = 0; k < 3; ++k) probe_fma8(x, fa, fb);
      probe_exp8(x);
    } else if constexpr (MODE == 3) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
    } else if constexpr (MODE == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) facc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ba, bb, facc[j], 0, 0, 0);
    } else if constexpr (MODE == 5) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
#pragma unroll
      for (int k = 0; k < 8; ++k) probe_fma8(x, fa, fb);
    } else if constexpr (MODE == 6) {
      if (first_on_simd) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) probe_fma8(x, fa, fb);
      }
    } else if constexpr (MODE == 7 || MODE == 12) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 3; ++k) probe_fma8(x, fa, fb);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (MODE == 12) __syncthreads();
    } else if constexpr (MODE == 8 || MODE == 9 || MODE == 10) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == 10) x[0] = __builtin_fmaf(x[0], fa, (float)acc[3][0]);
#pragma unroll
      for (int k = 0; k < 12; ++k) probe_fma8(x, fa, fb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE != 8) __syncthreads();
    } else if constexpr (MODE == 13 || MODE == 14) {
      const bool odd = MODE == 14 && ((wave >> 2) & 1);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        if ((half == 0) != odd) {
          // P: 4 groups of 4 MFMAs, each group followed by 32 fma
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < 4; ++k) probe_fma8(x, fa, fb);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
          // S: reads the last MFMA's result, then 25 x 8 fma and 4 x 8 exp
          x[0] = __builtin_fmaf(x[0], fa, (float)acc[3][0]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int f = 0; f < 6; ++f) probe_fma8(x, fa, fb);
            probe_exp8(x);
          }
          probe_fma8(x, fa, fb);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      __syncthreads();
    } else {
      const bool odd = (wave >> 2) & 1;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        if (odd == (half == 1)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa, qb, acc[j], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
          x[0] = __builtin_fmaf(x[0], fa, (float)acc[3][0]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 6; ++k) probe_fma8(x, fa, fb);
        __builtin_amdgcn_sched_barrier(0);
        if (half == 0) __syncthreads();
      }
      __syncthreads();
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float sink = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sink += x[i];
#pragma unroll
  for (int j = 0; j < 4; ++j) sink += (float)acc[j][lane & 15] + facc[j][lane & 15];
  if (lane == 0) {
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
    // (the sum joins the stored value only in a case no input produces, so nothing is optimised away)
    out[2 * w] = (int64_t)(t1 - t0) + (sink == 1234.5f ? 1 : 0);
    out[2 * w + 1] = (int64_t)(r1 - r0);
  }
}

}  // namespace tri
