// Tail growth of the decode cache (extension).
//
// The reference keeps every generated token in a bf16 tail of max_tail slots and, once it is full,
// overwrites the last slot (triattention/kernels/cuda/common_device.cuh:384).  Here, when the tail of a
// layer holds max_tail tokens, its oldest 64 tokens become one more tile of the quantized cache and the
// tail moves up by 64 slots:
//   * the tile is quantized as the prompt's tiles are, with the prompt's statistics: K centred by the
//     prompt's K mean, rotated and quantized with per-16-key-group scales (quantize_k_tile), V
//     normalised by the prompt's V mean and scale (pack_v_tile, clamped to the 8-bit range);
//   * it is classified as the newest tile of the cache (distance 0 from the end): state 8 for a q-head
//     whose band keeps at least one INT8 tile, else 4 for one that keeps an INT4 tile, else 0; the K
//     precision of the KV head is the maximum over its group and the rowmask the q-heads with state > 0
//     (decode.py:27-33 at d = 0); V is INT8 (the newest tiles are within NEAR_V8, decode.py:17-22).
//     A KV head that no q-head keeps drops the tile.  Exact (bf16) KV heads store it as KX/VX records;
//   * tiles already in the cache keep their classification, as the reference's cache never
//     reclassifies a stored tile.
// The host reserves room for `cap` such tiles per (sequence, KV head) and the slots they take (grow);
// the kernel runs at every decode step of the layer and spills only when the tail is full, so a
// captured decode step replays it unchanged.
#include "common.h"

namespace tri {

struct SpillArgs {
  const int64_t* step;  // tokens decoded since the store (the reference's step counter)
  int64_t* tail_base;   // [2]: tokens moved from the tail into the cache since the store; workgroups done
  uint16_t* ktail;      // [rows][hk][max_tail][128], strides tsb, tsh, tst
  uint16_t* vtail;
  int64_t tsb, tsh, tst;
  int max_tail, rows, hk, maxn, tiles_max, cap;
  // [rows][hk][4]: kinfo bits of the new tile (rowmask | INT4 K << 8; -1: no q-head keeps it), first K
  // record slot and first V record slot of the head's reserved run, task-table row of the head's first
  // growth split (-1: none)
  const int32_t* grow;
  const int32_t* prompt;  // [rows]
  const int32_t* xslot;   // [rows][hk]: first KX/VX record of an exact head, else -1 (may be null)
  int32_t* entry;         // [rows][hk][maxn]
  int32_t* kinfo;
  int32_t* slot;
  int32_t* count;  // [rows][hk]
  const int32_t* count0;  // [rows][hk]: count at the store (count <= count0 + tiles spilled since)
  int32_t* fmt;    // [rows][tiles_max]
  float* ka;       // [rows][hk][tiles_max][4]
  float* ka4;      // (may be null)
  const float* kstat;  // [rows][hk][3][128]
  const float* vstat;
  uint8_t* k8c;
  uint8_t* k4c;
  uint8_t* v8c;
  uint8_t* kxc;
  uint8_t* vxc;
  int64_t n_k8, n_k4, n_v8, n_kx;  // records each array holds
  int32_t* tasks;                  // decode task table (may be null)
  int n_tasks;
};

constexpr int SPILL_THREADS = 256;

// Whether every (sequence, KV head) has room for spilled tile k.  Each workgroup evaluates the whole
// launch's rule from arrays that no workgroup of the launch writes (prompt, grow, xslot, count0; the
// entry count of a head is at most count0 + k), so all of them reach the same answer before any row
// moves: without room anywhere, no tile is written, the tail and tail_base stay as they are and the
// tail clamps as the reference's does.
__device__ bool spill_has_room(const SpillArgs& a, int k) {
  bool ok = true;
  for (int p = threadIdx.x; p < a.rows * a.hk; p += SPILL_THREADS) {
    const int j = (a.prompt[p / a.hk] + BN - 1) / BN + k;
    ok = ok && j < a.tiles_max && a.count0[p] + k < a.maxn;
    const int x0 = a.xslot != nullptr ? a.xslot[p] : -1;
    const int4 gr = *reinterpret_cast<const int4*>(a.grow + (int64_t)p * 4);
    if (x0 >= 0) {
      ok = ok && (int64_t)x0 + j < a.n_kx;
    } else if (gr.x >= 0) {
      const bool is4 = (gr.x >> 8) & 1;
      ok = ok && (int64_t)gr.y + k < (is4 ? a.n_k4 : a.n_k8) && (int64_t)gr.z + k < a.n_v8 &&
           (!is4 || (a.k4c != nullptr && a.ka4 != nullptr));
    }
  }
  return __syncthreads_and(ok);
}

// One workgroup per (KV head, sequence).
__global__ __launch_bounds__(SPILL_THREADS) void tail_spill_kernel(SpillArgs a) {
  __shared__ __align__(16) union {
    struct {
      uint8_t c8[BN][D];
      uint8_t c4[BN][D];
      float vn[BN][D + 1];
    } q;
    uint16_t vt[BN * EXACT_VP];
  } sm;
  const int64_t tb = a.tail_base[0];
  if (*a.step - tb < a.max_tail) return;  // the tail has a free slot for this step's token
  const int k = (int)(tb / BN);           // tiles this cache has taken from the tail since the store
  if (k >= a.cap) return;                 // no room reserved: the tail clamps as the reference's does
  if (!spill_has_room(a, k)) return;      // (the same answer in every workgroup)
  const int kh = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int64_t hb = (int64_t)row * a.hk + kh;
  const int4 gr = *reinterpret_cast<const int4*>(a.grow + hb * 4);
  const int j = (a.prompt[row] + BN - 1) / BN + k;
  uint16_t* kt = a.ktail + row * a.tsb + kh * a.tsh;
  uint16_t* vt = a.vtail + row * a.tsb + kh * a.tsh;
  const int x0 = a.xslot != nullptr ? a.xslot[hb] : -1;
  const int e = a.count[hb];  // the new tile's entry
  if (j < a.tiles_max && e < a.maxn) {
    if (x0 >= 0) {
      const int64_t rec = (int64_t)x0 + j;
      if (rec < a.n_kx) {
        pack_exact_tile(kt, a.tst, vt, a.tst, BN, a.kxc + rec * KX_BYTES, a.vxc + rec * KX_BYTES, sm.vt);
        if (tid == 0) {
          a.entry[hb * a.maxn + e] = j | (1 << 30) | (1 << 29);
          a.kinfo[hb * a.maxn + e] = gr.x & 0xff;
          a.slot[hb * a.maxn + e] = 0;
          a.count[hb] = e + 1;
        }
      }
    } else if (gr.x >= 0) {
      const bool is4 = (gr.x >> 8) & 1;
      const int64_t ks = (int64_t)gr.y + k, vs = (int64_t)gr.z + k;
      if (ks < (is4 ? a.n_k4 : a.n_k8) && vs < a.n_v8 && (!is4 || (a.k4c != nullptr && a.ka4 != nullptr))) {
        float* kap = (is4 ? a.ka4 : a.ka) + (hb * a.tiles_max + j) * 4;
        quantize_k_tile(kt, a.tst, BN, a.kstat + hb * 3 * D, is4 ? nullptr : a.k8c + ks * K8_BYTES, kap,
                        is4 ? a.k4c + ks * K4_BYTES : nullptr, kap, sm.q.c8, sm.q.c4);
        const float* vm = a.vstat + hb * 3 * D;
        pack_v_tile(vt, a.tst, BN, vm, vm + 2 * D, nullptr, a.v8c + vs * V8_BYTES, nullptr, sm.q.vn);
        __syncthreads();  // the four group scales are written (lane 0 of each wave)
        if (tid == 0) {
          const int info = (gr.x & 0x1ff) | (int)((uint32_t)ks << 9);
          a.entry[hb * a.maxn + e] = j | (1 << 30) | (1 << 29);
          a.kinfo[hb * a.maxn + e] = info;
          a.slot[hb * a.maxn + e] = (int)vs;
          a.count[hb] = e + 1;
        }
        // the head's growth splits hold 64 entries each: entry k of the run is lane k % 64 of split k / 64
        const int tr = gr.w >= 0 ? gr.w + k / 64 : -1, lane = k % 64;
        if (a.tasks != nullptr && tr >= 0 && tr < a.n_tasks) {
          int32_t* t = a.tasks + (int64_t)tr * TASK_WORDS;
          if (tid == 0) {
            t[4 * lane] = (int)ks;
            t[4 * lane + 1] = (int)vs;
            t[4 * lane + 2] = (gr.x & 0x1ff) | (1 << 9) | (j << 10);
            if (lane > 0) t[4 * lane + 3] = lane + 1;
            t[4 * 1 + 3] = lane + 1;  // the split's entry count (lane 1's word; lane 0's holds the item)
          }
          if (tid < 4) reinterpret_cast<float*>(t)[256 + 4 * lane + tid] = kap[tid];
        }
      }
    }
    if (kh == 0 && tid == 0) a.fmt[(int64_t)row * a.tiles_max + j] = 1;
  }
  __syncthreads();  // the tile's rows are read
  // move tail rows [64, max_tail) to [0, max_tail - 64), 64 rows at a time: a chunk's rows are all read
  // before any of them is written over (the rows a chunk writes were read by the chunk before it)
  // (rows past the tail take the last row: those threads move it again, to the same slot)
  const int f = (tid & 15) * 8, rr = tid >> 4;  // this thread's feature offset and row within 16
  for (int r0 = BN; r0 < a.max_tail; r0 += BN) {
    const int r_0 = min(r0 + rr, a.max_tail - 1), r_1 = min(r0 + rr + 16, a.max_tail - 1);
    const int r_2 = min(r0 + rr + 32, a.max_tail - 1), r_3 = min(r0 + rr + 48, a.max_tail - 1);
    auto at = [&](uint16_t* base, int r) { return reinterpret_cast<uint4*>(base + (int64_t)r * a.tst + f); };
    const uint4 k0 = *at(kt, r_0), k1 = *at(kt, r_1), k2 = *at(kt, r_2), k3 = *at(kt, r_3);
    const uint4 v0 = *at(vt, r_0), v1 = *at(vt, r_1), v2 = *at(vt, r_2), v3 = *at(vt, r_3);
    __syncthreads();
    *at(kt, r_0 - BN) = k0;
    *at(kt, r_1 - BN) = k1;
    *at(kt, r_2 - BN) = k2;
    *at(kt, r_3 - BN) = k3;
    *at(vt, r_0 - BN) = v0;
    *at(vt, r_1 - BN) = v1;
    *at(vt, r_2 - BN) = v2;
    *at(vt, r_3 - BN) = v3;
  }
  // the last workgroup to finish moves the tail base (every workgroup has read it by then)
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const unsigned long long done = atomicAdd(reinterpret_cast<unsigned long long*>(a.tail_base + 1), 1ull);
    if (done == (unsigned long long)gridDim.x * gridDim.y - 1) {
      a.tail_base[0] = tb + BN;
      a.tail_base[1] = 0;
    }
  }
}

}  // namespace tri
