// Decode-cache assembly on the device: the kept-tile metadata of one Prefill call's batch and the
// compaction of its records into the cache's arrays.
//
// Reference semantics: triattention/kernels/decode.py:24-67 (DecodeCache.store), which classifies the
// tiles and compacts the records on the host with torch.  The rules are its own:
//   * state of tile j for a q-head with band (w8, w4): 8 if j == 0 or d < w8, 4 if d < w4, else 0,
//     with d = tiles - 1 - j (decode.py:27-30);
//   * K precision of a (KV head, tile): the maximum state over the head's GQA group; the tile is kept
//     when that is > 0, and its rowmask has bit r set when q-head r of the group has state > 0
//     (decode.py:31-33);
//   * kept tiles of a head are listed in ascending order (decode.py:36); INT4 and INT8 K records, and
//     INT8 and INT4 V records, are each numbered in (KV head, entry) order (decode.py:38-53);
//   * V is INT8 for the sink tile and the last NEAR_V8 tiles, INT4 elsewhere (decode.py:17-22).
// Extension: KV heads kept exact (bf16) keep every tile with every q-head's bit set, select no quantized
// record, and copy their KX / VX records whole.
//
// One workgroup per (tile chunk, KV head, sequence).  Every workgroup classifies the tiles of every KV
// head of its sequence (a few thousand state evaluations) and scans them, so it knows each of its tiles'
// entry index and record slots without any other workgroup; the chunk-0 workgroup of a head writes the
// head's metadata row, and every workgroup copies the records of its chunk's kept tiles with coalesced
// 16-byte accesses.
#include "common.h"

namespace tri {

constexpr int STORE_CHUNK = 16;    // tiles whose records one workgroup copies
constexpr int STORE_THREADS = 256;
constexpr int STORE_MAX_HQ = 256;  // q-heads whose bands the kernel stages in LDS

struct CacheStoreArgs {
  const int32_t* bands;  // [hq][2] (w8, w4)
  const int32_t* exact;  // [hk]: -1 for a quantized KV head, else its slot among the exact heads; may be null
  int hq, hk, t, tiles, nx, batch;
  int xstride;  // records per (sequence, exact head) in the destination (>= tiles: room for tail tiles)
  // sources: the Prefill call's outputs, [batch][hk][tiles] records and scales
  const uint8_t* kp;   // K8
  const uint8_t* k4p;  // K4 (may be null when no tile is INT4)
  const uint8_t* v8p;
  const uint8_t* v4p;  // (may be null when no tile has INT4 V)
  const uint8_t* kx;   // [batch][nx][tiles] KX / VX records of the exact heads (may be null)
  const uint8_t* vx;
  const float* ka;     // [batch][hk][tiles][4]
  const float* ka4;    // (may be null)
  const float* kstat;  // [batch][hk][3][128]
  const float* vstat;
  // destination: rows row0 .. row0 + batch - 1 of the cache (rows allocated: `rows`)
  int row0, rows, maxn, tiles_max;
  int32_t* entry;  // [rows][hk][maxn]
  int32_t* kinfo;
  int32_t* slot;
  int32_t* count;  // [rows][hk]
  int32_t* fmt;    // [rows][tiles_max]
  int32_t* prompt; // [rows]
  int32_t* xslot;  // [rows][hk] (may be null when no head is exact)
  float* ka_c;     // [rows][hk][tiles_max][4]
  float* ka4_c;    // (may be null)
  float* kstat_c;  // [rows][hk][3][128]
  float* vstat_c;
  uint8_t* k8c;    // compacted record arrays, first free record o*, records held cap*
  uint8_t* k4c;
  uint8_t* v8c;
  uint8_t* v4c;
  uint8_t* kxc;
  uint8_t* vxc;
  int64_t o8, o4, ov8, ov4, ox;
  int64_t cap8, cap4, capv8, capv4, capx;
};

// counts of one tile packed in 12-bit fields: kept | INT4 K << 12 | INT8 K << 24 | INT8 V << 36 | INT4 V << 48
__device__ __forceinline__ uint64_t tile_counts(bool kept, bool is4, bool is8, bool v8, bool v4) {
  return (uint64_t)kept | (uint64_t)is4 << 12 | (uint64_t)is8 << 24 | (uint64_t)v8 << 36 | (uint64_t)v4 << 48;
}
__device__ __forceinline__ int field(uint64_t c, int f) { return (int)((c >> (12 * f)) & 0xfffu); }

struct TileClass {
  bool kept, is4, is8, v8, v4;
  int mask;
};

__device__ __forceinline__ TileClass classify(const int* sb, int g, bool ex, int tiles, int j) {
  TileClass c;
  int kv = 0, mask = 0;
  const int d = tiles - 1 - j;
#pragma unroll 1
  for (int r = 0; r < g; ++r) {
    const int w8 = sb[2 * r], w4 = sb[2 * r + 1];
    const int s = ex ? 8 : (j == 0 || d < w8) ? 8 : (d < w4 ? 4 : 0);
    kv = max(kv, s);
    mask |= (s > 0 ? 1 : 0) << r;
  }
  const bool vi8 = j == 0 || d < NEAR_V8;
  c.kept = kv > 0;
  c.is4 = !ex && kv == 4;
  c.is8 = !ex && kv == 8;
  c.v8 = !ex && c.kept && vi8;
  c.v4 = !ex && c.kept && !vi8;
  c.mask = mask;
  return c;
}

// exclusive prefix (this thread's) and total of v over the workgroup, in thread order
__device__ __forceinline__ uint64_t block_scan(uint64_t v, uint64_t& total, uint64_t* lds) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint64_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint64_t o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) lds[w] = inc;
  __syncthreads();
  uint64_t before = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < STORE_THREADS / 64; ++i) {
    if (i < w) before += lds[i];
    total += lds[i];
  }
  __syncthreads();
  return before + inc - v;
}

struct CopyDesc {
  int64_t ksrc, kdst, vsrc, vdst;  // record indices (-1: nothing to copy)
  int kbytes, vbytes;
  int kind;  // 0 quantized K and V, 1 exact KX and VX
};

__global__ __launch_bounds__(STORE_THREADS) void cache_store_kernel(CacheStoreArgs a) {
  __shared__ int sb[2 * STORE_MAX_HQ];
  __shared__ uint64_t scan_lds[STORE_THREADS / 64];
  __shared__ CopyDesc desc[STORE_CHUNK];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.x, kh = blockIdx.y, s = blockIdx.z;
  const int g = a.hq / a.hk, tiles = a.tiles, row = a.row0 + s;
  for (int i = tid; i < 2 * a.hq; i += STORE_THREADS) sb[i] = a.bands[i];
  if (tid < STORE_CHUNK) desc[tid] = CopyDesc{0, 0, 0, 0, 0, 0, 0};
  __syncthreads();
  // this thread's run of tiles: [j0, j1)
  const int run = (tiles + STORE_THREADS - 1) / STORE_THREADS;
  const int j0 = min(tiles, tid * run), j1 = min(tiles, j0 + run);
  // counts of the heads before kh (record numbering is (KV head, entry) order within a sequence), the
  // sequence's totals (plain ints: summed over heads they outgrow the 12-bit packed fields), and this
  // thread's prefix within head kh
  int before_head[5] = {0, 0, 0, 0, 0}, seq_total[5] = {0, 0, 0, 0, 0};
  uint64_t my_prefix = 0, head_total = 0;
  for (int h = 0; h < a.hk; ++h) {
    const bool ex = a.exact != nullptr && a.exact[h] >= 0;
    uint64_t mine = 0;
    for (int j = j0; j < j1; ++j) {
      const TileClass c = classify(sb + 2 * h * g, g, ex, tiles, j);
      mine += tile_counts(c.kept, c.is4, c.is8, c.v8, c.v4);
    }
    uint64_t total;
    const uint64_t pre = block_scan(mine, total, scan_lds);
    if (h == kh) {
      my_prefix = pre;
      head_total = total;
    }
#pragma unroll
    for (int f = 0; f < 5; ++f) {
      if (h < kh) before_head[f] += field(total, f);
      seq_total[f] += field(total, f);
    }
  }
  const bool ex = a.exact != nullptr && a.exact[kh] >= 0;
  const int xs = ex ? a.exact[kh] : 0;
  const int64_t hb_src = (int64_t)s * a.hk + kh;
  const int64_t hb = (int64_t)row * a.hk + kh;
  const bool writer = chunk == 0 && row < a.rows;
  // walk this thread's tiles with the running counts: entry index and record slots
  int run_pre[5];  // counts before the current tile, within the sequence
#pragma unroll
  for (int f = 0; f < 5; ++f) run_pre[f] = before_head[f] + field(my_prefix, f);
  int e = field(my_prefix, 0);  // entry index of this thread's first kept tile in head kh
  for (int j = j0; j < j1; ++j) {
    const TileClass c = classify(sb + 2 * kh * g, g, ex, tiles, j);
    if (c.kept) {
      const int64_t k4slot = a.o4 + (int64_t)s * seq_total[1] + run_pre[1];
      const int64_t k8slot = a.o8 + (int64_t)s * seq_total[2] + run_pre[2];
      const int64_t v8slot = a.ov8 + (int64_t)s * seq_total[3] + run_pre[3];
      const int64_t v4slot = a.ov4 + (int64_t)s * seq_total[4] + run_pre[4];
      const int64_t kslot = c.is4 ? k4slot : c.is8 ? k8slot : 0;
      const int64_t vslot = c.v8 ? v8slot : c.v4 ? v4slot : 0;
      if (writer && e < a.maxn) {
        const bool vi8 = j == 0 || tiles - 1 - j < NEAR_V8;
        a.entry[hb * a.maxn + e] = j | (1 << 30) | (vi8 ? 1 << 29 : 0);
        a.kinfo[hb * a.maxn + e] = (c.mask & 0xff) | (c.is4 ? 1 << 8 : 0) | (int)((uint32_t)kslot << 9);
        a.slot[hb * a.maxn + e] = (int)vslot;
      }
      if (j / STORE_CHUNK == chunk) {
        CopyDesc dsc;
        if (ex) {
          const int64_t src = ((int64_t)s * a.nx + xs) * tiles + j;
          const int64_t dst = a.ox + ((int64_t)s * a.nx + xs) * a.xstride + j;
          dsc.kind = 1;
          dsc.ksrc = dsc.vsrc = src;
          dsc.kdst = dsc.vdst = dst;
          dsc.kbytes = dsc.vbytes = dst < a.capx ? KX_BYTES : 0;
        } else {
          dsc.kind = 0;
          dsc.ksrc = hb_src * tiles + j;
          dsc.kdst = kslot;
          dsc.kbytes = c.is4 ? (k4slot < a.cap4 ? K4_BYTES : 0) : (k8slot < a.cap8 ? K8_BYTES : 0);
          dsc.vsrc = hb_src * tiles + j;
          dsc.vdst = vslot;
          dsc.vbytes = c.v8 ? (v8slot < a.capv8 ? V8_BYTES : 0) : (v4slot < a.capv4 ? V4_BYTES : 0);
          if (c.is4 && a.k4p == nullptr) dsc.kbytes = 0;
          if (c.v4 && a.v4p == nullptr) dsc.vbytes = 0;
        }
        desc[j % STORE_CHUNK] = dsc;
      }
      ++e;
    }
    run_pre[0] += c.kept;
    run_pre[1] += c.is4;
    run_pre[2] += c.is8;
    run_pre[3] += c.v8;
    run_pre[4] += c.v4;
  }
  if (writer) {
    const int cnt = field(head_total, 0);
    for (int i = cnt + tid; i < a.maxn; i += STORE_THREADS) {
      a.entry[hb * a.maxn + i] = 0;
      a.kinfo[hb * a.maxn + i] = 0;
      a.slot[hb * a.maxn + i] = 0;
    }
    if (tid == 0) {
      a.count[hb] = cnt;
      if (a.xslot) a.xslot[hb] = ex ? (int)(a.ox + ((int64_t)s * a.nx + xs) * a.xstride) : -1;
    }
    for (int i = tid; i < a.tiles_max * 4; i += STORE_THREADS) {
      a.ka_c[hb * a.tiles_max * 4 + i] = i < tiles * 4 ? a.ka[hb_src * tiles * 4 + i] : 1.f;
      if (a.ka4_c) a.ka4_c[hb * a.tiles_max * 4 + i] = (i < tiles * 4 && a.ka4) ? a.ka4[hb_src * tiles * 4 + i] : 1.f;
    }
    for (int i = tid; i < 3 * D; i += STORE_THREADS) {
      a.kstat_c[hb * 3 * D + i] = a.kstat[hb_src * 3 * D + i];
      a.vstat_c[hb * 3 * D + i] = a.vstat[hb_src * 3 * D + i];
    }
    if (kh == 0) {
      if (tid == 0) a.prompt[row] = a.t;
      for (int j = tid; j < a.tiles_max; j += STORE_THREADS)
        a.fmt[(int64_t)row * a.tiles_max + j] = (j < tiles && !(j == 0 || tiles - 1 - j < NEAR_V8)) ? 2 : 1;
    }
  }
  __syncthreads();
  // copy the chunk's kept records, one tile after another, 16 bytes per thread per step
  const int nt = min(STORE_CHUNK, tiles - chunk * STORE_CHUNK);
  for (int i = 0; i < nt; ++i) {
    const CopyDesc d = desc[i];
    const uint8_t* ks = d.kind ? a.kx + d.ksrc * KX_BYTES
                               : (d.kbytes == K4_BYTES ? a.k4p + d.ksrc * K4_BYTES : a.kp + d.ksrc * K8_BYTES);
    uint8_t* kd = d.kind ? a.kxc + d.kdst * KX_BYTES
                         : (d.kbytes == K4_BYTES ? a.k4c + d.kdst * K4_BYTES : a.k8c + d.kdst * K8_BYTES);
    for (int off = tid * 16; off < d.kbytes; off += STORE_THREADS * 16)
      *reinterpret_cast<uint4*>(kd + off) = *reinterpret_cast<const uint4*>(ks + off);
    const uint8_t* vs = d.kind ? a.vx + d.vsrc * KX_BYTES
                               : (d.vbytes == V4_BYTES ? a.v4p + d.vsrc * V4_BYTES : a.v8p + d.vsrc * V8_BYTES);
    uint8_t* vd = d.kind ? a.vxc + d.vdst * KX_BYTES
                         : (d.vbytes == V4_BYTES ? a.v4c + d.vdst * V4_BYTES : a.v8c + d.vdst * V8_BYTES);
    for (int off = tid * 16; off < d.vbytes; off += STORE_THREADS * 16)
      *reinterpret_cast<uint4*>(vd + off) = *reinterpret_cast<const uint4*>(vs + off);
  }
}

}  // namespace tri
