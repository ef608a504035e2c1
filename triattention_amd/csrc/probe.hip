// Streaming-read probe: the HBM read rate a kernel with no compute reaches on this device, for a
// given byte count and launch shape.  It is the practical ceiling the split-KV decode kernel's
// record stream is compared against (the decode kernel reads each record once, in 1 KiB
// fragments of 16 bytes per lane, as this probe does).  No reference counterpart.
#include "common.h"

namespace tri {

constexpr int PROBE_RECORD = 8192;  // bytes per record (a K8 / V8 record)

// Wave i reads records [i * per, (i + 1) * per) in order, DEPTH records in flight: eight 16-byte
// loads per lane per record, through a descriptor per record (loads past the array read zeros
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
    for (int f = 0; f < 8; ++f) buf[d][f] = __builtin_amdgcn_raw_buffer_load_b128(rs, L * 16 + f * 1024, 0, 0);
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
