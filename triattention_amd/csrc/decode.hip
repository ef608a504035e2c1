// Split-KV decode over the quantized cache, plus the merge with the bf16 tail.
//
// Reference semantics: triattention/kernels/cuda/common_device.cuh:178-469
// (decode_tile, decode_kernel, decode_merge_kernel) and the cache metadata of
// triattention/kernels/decode.py:24-67.
//
// One 64-lane wave per (sequence, KV head, split).  The kept tiles of a split
// stream straight from HBM into MFMA operand registers (one 16-byte load per
// lane per 1 KiB fragment, the next tile's K and V issued while the current one
// is processed); no LDS staging is needed because every fragment is consumed by
// exactly one wave.  Quantized heads: the g <= 8 query heads of the KV group
// are the rows of the MFMA A operand (S = Q K^T, one key per lane and row
// block); with groups of up to 4 and 4-bit keys, each lane instead scores its
// own key against the group's rows with packed 4-bit dot products
// (v_dot8_i32_i4, the same integers); exact heads: the q-heads are the columns
// of the B operand (S^T = K Q^T).
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
  int64_t n_k8, n_k4, n_v8, n_v4;  // records in the compacted arrays
  // exact (bf16) KV heads: xslot[B][Hk] = first KX/VX record of the (sequence,
  // KV head) whose tiles are all kept (record of tile j at xslot + j), or -1
  // for a quantized head; xslot may be null when no head is exact
  const int32_t* xslot;
  const uint8_t* kxc;
  const uint8_t* vxc;
  const float* kstat;   // [B][Hk][3][128]: K mean (the frame of the merge's tail scores)
  const float* vstat;   // [B][Hk][3][128]: V mean, scale, 1/scale
  int64_t n_kx;
  // work scatter: the grid is 1-D with `launched` = items | 1 workgroups (odd); workgroup lin takes work
  // item lin * scatter mod launched (a permutation), and the one padding item (>= items) exits
  int64_t scatter;
  int items, launched;
  int64_t total;  // work items of the cache layout: splits x hk x batch (a task row naming another is padding)
  // split partition (extension): null for the reference's uniform split of `per` tiles, else
  // [B][Hk][splits + 1] entry bounds, split s of a head covering entries [bounds[s], bounds[s + 1])
  const int32_t* bounds;
  // task table (extension, may be null): 512 int32 words per listed work item (sequence, KV head,
  // split): int4 (K record offset, V record offset, flags, w) for lanes 0..63 with w the work item in
  // lane 0 and the split's entry count in the others, then float4 K group scales for lanes 0..63
  // (decode_tasks_kernel).  The launch then covers the listed items only (`items` of them).
  const int32_t* tasks;
};

constexpr int MAX_TAIL = 1024;
// the merge's one-wave form: grids of at least SHORT_WIDE (sequence, q-head) workgroups per CU
constexpr int SHORT_WIDE = 2;
// entry words: bits 0-28 the tile index; bit 30 set (extension) marks that bit 29 holds the
// tile's V format (1 = INT8 V), so the kernel need not read fmt for it
constexpr int ENTRY_TILE = (1 << 29) - 1, ENTRY_V8 = 1 << 29, ENTRY_VFMT = 1 << 30;
constexpr int MAX_PER = 64;  // kept tiles per split: one per lane of the wave's metadata

// Entries [first, last) of split `split` of head hb: the uniform split of a.per
// tiles, or the caller's partition clamped into [0, count) and to MAX_PER
// entries (a partition outside that contract loses tiles, never reads out of
// bounds).
__device__ __forceinline__ void split_range(const DecodeArgs& a, int64_t hb, int split, int& first, int& last) {
  const int cnt = a.count[hb];
  if (a.bounds) {
    const int32_t* bd = a.bounds + hb * (a.splits + 1) + split;
    first = min(max(bd[0], 0), cnt);
    last = min(max(bd[1], first), min(cnt, first + MAX_PER));
  } else {
    first = split * a.per;
    last = min(cnt, first + a.per);
  }
}

constexpr int NO_RECORD = -1;  // the record slot of an entry past a split's end (its loads read zeros)

// Buffer descriptor of record `slot` (`bytes` long) of an array of n records: loads through it at
// offsets past the record, or through the descriptor of a slot outside the array (num_records 0),
// return zeros without touching memory.  Each record gets its own 64-bit base, so the arrays may
// exceed the 32-bit offsets of a single descriptor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t record_rsrc(const uint8_t* base, int slot, int64_t n, int bytes) {
  const bool ok = slot >= 0 && slot < n;
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)(ok ? slot : 0) * bytes), (short)0,
                                           ok ? bytes : 0, 0x00020000);
}
constexpr int TASK_WORDS = 512;

// Task table of the split kernel (extension): lane L of work item (sequence, KV head, split) gets
// entry first + L of the split -- its K and V record slots, rowmask | INT4-K << 8 | INT8-V << 9
// | tile << 10, the split's entry count, and the tile's four K group scales.  The split kernel then
// starts streaming a split's records one memory round trip after it starts, instead of three (split
// bounds, then entry / kinfo / slot, then the records).  Built once per cache layout: the entries and
// the split partition change only when the cache is stored.
__global__ __launch_bounds__(64) void decode_tasks_kernel(DecodeArgs a, const int32_t* items, int32_t* tasks) {
  const int L = threadIdx.x;
  const int item = items ? items[blockIdx.x] : (int)blockIdx.x;
  int32_t* t = tasks + (int64_t)blockIdx.x * TASK_WORDS;
  if (item < 0 || item >= a.total) {
    // an item outside the layout: an empty row (no entry, no record) whose work item -1 marks it as
    // padding for the split kernel
    *reinterpret_cast<int4*>(t + 4 * L) = make_int4(NO_RECORD, NO_RECORD, 1 << 9, L == 0 ? -1 : 0);
    *reinterpret_cast<float4*>(t + 256 + 4 * L) = make_float4(1.f, 1.f, 1.f, 1.f);
    return;
  }
  const int split = item % a.splits, kh = (item / a.splits) % a.hk, b = item / (a.splits * a.hk);
  const int64_t hb = (int64_t)b * a.hk + kh;
  int first, last;
  split_range(a, hb, split, first, last);
  const int n = max(0, last - first);
  int4 w = make_int4(NO_RECORD, NO_RECORD, 1 << 9, L == 0 ? item : n);
  float4 ks = make_float4(1.f, 1.f, 1.f, 1.f);
  if (L < n) {
    const int64_t li = hb * a.maxn + min(first + L, a.maxn - 1);
    const int info = a.kinfo[li], er = a.entry[li], vs = a.slot[li];
    const int is4 = (info >> 8) & 1;
    const int j = min(max(er & ENTRY_TILE, 0), a.tiles_max - 1);
    const int vf = (er & ENTRY_VFMT) ? ((er & ENTRY_V8) ? 1 : 2) : a.fmt[(int64_t)b * a.tiles_max + j];
    w.x = (int)((unsigned)info >> 9);
    w.y = vs;
    w.z = (info & 0x1ff) | ((vf == 1) << 9) | (j << 10);
    ks = *reinterpret_cast<const float4*>(((is4 && a.ka4) ? a.ka4 : a.ka) + (hb * a.tiles_max + j) * 4);
  }
  *reinterpret_cast<int4*>(t + 4 * L) = w;
  *reinterpret_cast<float4*>(t + 256 + 4 * L) = ks;
}

// The empty split partial (m = -FLT_MAX, l = 0, o = 0) for n (q-head, split) slots: the partials of the
// splits a task table leaves out (they hold no kept tile).
__global__ __launch_bounds__(256) void fill_empty_partials_kernel(float* pm, float* pl, float* po, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    pm[i] = -3.402823466e38f;
    pl[i] = 0.f;
  }
  for (int64_t k = i; k < n * D; k += (int64_t)gridDim.x * 256) po[k] = 0.f;
}

__device__ __forceinline__ v4i unpack16(v4i w) {
  return v4i{(int)nib_lo16((uint32_t)w[0]), (int)nib_hi16((uint32_t)w[0]), (int)nib_lo16((uint32_t)w[1]),
             (int)nib_hi16((uint32_t)w[1])};
}

// Split partials of an exact (bf16) KV head over its prompt tiles [first, last):
// S^T = K Q^T with bf16 MFMA (the g q-heads are the columns), scores
// (q.k - q.kmean) * sm_log2 in the frame of the merge's tail scores, fp32 online
// softmax, P split into bf16 high and low parts, O^T = V^T P^T.  The partials
// use the quantized heads' convention: m in log2 units, l = sum p, o = sum p v'
// with v' = (v - mean) / scale, so the merge treats every head alike.
__device__ __forceinline__ void decode_exact(const DecodeArgs& a, int b, int kh, int split) {
  // Q as the B operand, kept in LDS: column lq = q-head kh*g + lq, features ks*16 + 8*half + e
  __shared__ __align__(16) uint16_t qx[32][D];
  const int L = threadIdx.x, lq = L & 31, half = L >> 5;
  const int g = a.hq / a.hk, prompt = a.prompt[b], ptiles = (prompt + BN - 1) / BN;
  const int64_t hb = (int64_t)b * a.hk + kh;
  int first, last;
  split_range(a, hb, split, first, last);
  const int x0 = a.xslot[hb];
  float cq = 0.f;
  const float* kmean = a.kstat + hb * 3 * D;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    uint4 w = make_uint4(0, 0, 0, 0);
    if (lq < g) w = *reinterpret_cast<const uint4*>(a.q + b * a.qsb + (int64_t)(kh * g + lq) * a.qsh + ks * 16 + 8 * half);
    *reinterpret_cast<uint4*>(&qx[lq][ks * 16 + 8 * half]) = w;
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      cq = __builtin_fmaf(bf16f((ww[e >> 1] >> (16 * (e & 1))) & 0xffffu), kmean[ks * 16 + 8 * half + e], cq);
  }
  cq += __shfl_xor(cq, 32, 64);
  __syncthreads();
  v16f acc[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[cb][r] = 0.f;
  float m = -3.402823466e38f, den = 0.f;
  v4i kf[8], vf[8];
  // half step hs covers keys 32*(hs & 1) .. +31 of tile first + hs / 2 (record x0 + tile); the
  // next half's K streams in after the QK MFMAs, its V after the PV MFMAs
  auto load_k = [&](int hs) {
    const __amdgpu_buffer_rsrc_t rk = record_rsrc(a.kxc, x0 + first + (hs >> 1), a.n_kx, KX_BYTES);
#pragma unroll
    for (int F = 0; F < 8; ++F)
      kf[F] = __builtin_amdgcn_raw_buffer_load_b128(rk, L * 16 + F * 1024, (hs & 1) * (KX_BYTES / 2), LOAD_STREAM);
  };
  auto load_v = [&](int hs) {
    const __amdgpu_buffer_rsrc_t rv = record_rsrc(a.vxc, x0 + first + (hs >> 1), a.n_kx, KX_BYTES);
#pragma unroll
    for (int F = 0; F < 8; ++F)
      vf[F] = __builtin_amdgcn_raw_buffer_load_b128(rv, L * 16 + F * 1024, (hs & 1) * (KX_BYTES / 2), LOAD_STREAM);
  };
  const int steps = 2 * max(0, last - first);
  if (steps > 0) {
    load_k(0);
    load_v(0);
  }
  for (int hs = 0; hs < steps; ++hs) {
    v16f sc = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      sc = mfma_bf16(__builtin_bit_cast(v8bf, kf[ks]), *reinterpret_cast<const v8bf*>(&qx[lq][ks * 16 + 8 * half]),
                     sc);
    if (hs + 1 < steps) load_k(hs + 1);
    const int key0 = (first + (hs >> 1)) * BN + (hs & 1) * 32;
    // keys past the prompt exist only in its last tile; tiles after it (spilled from the tail) are full
    const int lim = first + (hs >> 1) < ptiles ? prompt : INT_MAX;
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
      sc[r] = key < lim ? (sc[r] - cq) * a.sm_log2 : -__builtin_inff();
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float n = fmaxf(m, mx), alpha = __builtin_amdgcn_exp2f(m - n);
    m = n;
    den *= alpha;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[cb][r] *= alpha;
    v8bf phi[2], plo[2];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = __builtin_amdgcn_exp2f(sc[r] - n);
      const __bf16 h = (__bf16)p;
      phi[r >> 3][r & 7] = h;
      plo[r >> 3][r & 7] = (__bf16)(p - (float)h);
      psum += p;
    }
    den += psum + __shfl_xor(psum, 32, 64);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int kh2 = 0; kh2 < 2; ++kh2) {
        const v8bf v = __builtin_bit_cast(v8bf, vf[cb * 2 + kh2]);
        acc[cb] = mfma_bf16(v, phi[kh2], acc[cb]);
        acc[cb] = mfma_bf16(v, plo[kh2], acc[cb]);
      }
    if (hs + 1 < steps) load_v(hs + 1);
  }
  if (lq >= g) return;
  const int64_t idx = ((int64_t)b * a.hq + kh * g + lq) * a.splits + split;
  const float* vmean = a.vstat + hb * 3 * D;
  const float* vinv = vmean + 2 * D;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int ch = cb * 32 + 8 * r4 + 4 * half;
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (acc[cb][r4 * 4 + i] - vmean[ch + i] * den) * vinv[ch + i];
      *reinterpret_cast<float4*>(a.po + idx * D + ch) = make_float4(o[0], o[1], o[2], o[3]);
    }
  if (half == 0) {
    a.pl[idx] = den;
    a.pm[idx] = m;
  }
}

// R: q-head rows per lane half (min(group, 4)); EXACT: the launch holds exact
// (bf16) KV heads, whose path is compiled in only then (it needs 2 waves/SIMD).
// DUP (groups of at most 4 q-heads): the score rows 4..7 of the QK MFMA do not
// exist, so the upper half of the wave takes the tile's second 32-key block
// for rows 0..3 instead, and every lane carries R scores rather than 2R.
// NW: waves per workgroup.  With NW = 2 the two waves share the split's Q
// quantization and metadata, take its tiles alternately (wave w: entries first
// + w, first + w + 2, ...), and combine their running (m, l, o) in LDS at the
// end, so that each SIMD holds two waves whose dependency chains interleave.
// TASKS: the launch has a task table (a.tasks, quantized heads only), whose rows give each split's
// entries; a separate instantiation, so that the common path has no branch between the first
// tile's record loads and the use of Q (at a join of two paths the compiler waits for every
// outstanding load, which would hold the Q quantization until the records arrive).
template <int R, bool EXACT = false, bool DUP = false, int NW = 1, int W = 2, bool TASKS = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(W))) void decode_kernel(DecodeArgs a) {
  static_assert(NW == 1 || (NW == 2 && !EXACT), "two waves per workgroup only for quantized heads");
  static_assert(!(TASKS && EXACT), "task tables list quantized heads only");
  __shared__ __align__(16) int8_t q8s[MAX_GROUP][D];
  __shared__ __align__(16) int8_t q4s[MAX_GROUP][D];
  __shared__ float qsc[MAX_GROUP], qsc4[MAX_GROUP];
  __shared__ __align__(16) uint32_t q4w[MAX_GROUP][D / 8];  // packed 4-bit Q words (DUP score path)
  __shared__ __align__(16) uint8_t pls_all[NW][MAX_GROUP][BN];
  __shared__ __align__(16) int4 meta[MAX_PER + 1];     // per-tile record offsets and flags
  __shared__ __align__(16) float4 metk[MAX_PER + 1];   // per-tile K group scales

  // Workgroups are dealt to the 8 XCDs round-robin by linear id.  Work item w = lin * scatter mod
  // launched spreads each head's splits over the XCDs and CUs (the host picks the multiplier, and a
  // golden-ratio one with an odd launch count where a plain one would pin split indices to XCDs).
  // Splits share no data but Q, so nothing is lost in L2.
  int split, kh, b;
  int first, last;
  int4 task_w = make_int4(0, 0, 0, 0);
  float4 task_k = make_float4(1.f, 1.f, 1.f, 1.f);
  {
    const int w = (int)(((int64_t)blockIdx.x * a.scatter) % a.launched);
    if (w >= a.items) return;  // the padding item (whole workgroup, before any barrier)
    int item = w;
    if constexpr (TASKS) {
      // w-th listed split: its work item, entry count and every entry the prologue needs
      const int32_t* t = a.tasks + (int64_t)w * TASK_WORDS;
      task_w = *reinterpret_cast<const int4*>(t + 4 * (threadIdx.x & 63));
      task_k = *reinterpret_cast<const float4*>(t + 256 + 4 * (threadIdx.x & 63));
      item = __builtin_amdgcn_readlane(task_w.w, 0);
      // (a row naming no work item of this layout -- the builder's padding row, or a stale or foreign
      // table -- is padding too; the entry count is clamped to one wave's metadata)
      if (item < 0 || item >= a.total) return;
      first = 0;
      last = min(max(__builtin_amdgcn_readlane(task_w.w, 1), 0), MAX_PER);
    }
    const int nsplit = a.splits, nkh = a.hk;
    split = item % nsplit;
    kh = (item / nsplit) % nkh;
    b = item / (nsplit * nkh);
  }
  // A split past its head's kept tiles (ragged batches: most splits of the short sequences)
  // writes the empty partial (m = -FLT_MAX, l = 0, o = 0) and leaves.
  const int wv = NW > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;
  if constexpr (!TASKS) split_range(a, (int64_t)b * a.hk + kh, split, first, last);
  if (first >= last) {
    if (wv) return;
    const int L = threadIdx.x & 63, g = a.hq / a.hk;
    for (int r = 0; r < g; ++r) {
      const int64_t idx = ((int64_t)b * a.hq + kh * g + r) * a.splits + split;
      *reinterpret_cast<float2*>(a.po + idx * D + 2 * L) = make_float2(0.f, 0.f);
      if (L == 0) {
        a.pm[idx] = -3.402823466e38f;
        a.pl[idx] = 0.f;
      }
    }
    return;
  }
  if constexpr (EXACT) {
    if (a.xslot[(int64_t)b * a.hk + kh] >= 0) {
      decode_exact(a, b, kh, split);
      return;
    }
  }
  const int L = threadIdx.x & 63, lq = L & 31, half = L >> 5;
  const int g = a.hq / a.hk;
  const int prompt = a.prompt[b], ptiles = (prompt + BN - 1) / BN;
  uint8_t (&pls)[MAX_GROUP][BN] = pls_all[wv];
  const int64_t hb = (int64_t)b * a.hk + kh;

  // The g query rows are loaded first, one row per 8 lanes, 16 channels per
  // lane (the padding rows load row g - 1, so every lane issues the same
  // loads); quantization waits for them only after the first tile's record
  // loads are in flight.
  const int qrw = L >> 3, qt = L & 7;
  uint2 qraw[4];
  {
    const uint16_t* qp = a.q + b * a.qsb + (int64_t)(kh * g + min(qrw, g - 1)) * a.qsh + qt * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) qraw[i] = *reinterpret_cast<const uint2*>(qp + 4 * i);
  }
  // rows of this lane: 4*half + r (r < R), or r with DUP; the owner row of this
  // lane's scalar work: 4*half + (L & 3), or L & 3 with DUP (lower half writes it)
  constexpr int NK = DUP ? 1 : 2;  // 32-key blocks per lane
  const int orow = DUP ? (L & 3) : 4 * half + (L & 3);
  const bool owner = (L & 3) < R && (!DUP || half == 0);
  auto qrow = [&](int r) { return DUP ? r : 4 * half + r; };
  float m_o = -3.402823466e38f;
  float den[R], acc[4][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    den[r] = 0.f;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[cb][r] = 0.f;
  }
  const int64_t mbase = hb * a.maxn;
  // Record streams are read through one buffer descriptor per record (record_rsrc: uniform 64-bit
  // base, 32-bit lane offsets); a slot outside its array, or an offset past its record, reads zeros.
  // The loads are non-temporal (LOAD_STREAM): every record is read once per step, and with the
  // default policy the stream displaced what the split and merge kernels reread (C1 split kernel
  // 35.9 -> 33.2 us, decode op 43.3 -> 39.5 us, C3 split kernel 104 -> 93 us, same box).
  v4i kf[8], vf8[8];
  float kav[2], kmax = 0.f;
  // Per-tile metadata of this split in LDS: lane L loads entry first + L with
  // vector loads in the prologue (at most 64 entries per split; entries past
  // the end hold record offsets beyond every record array, whose loads return
  // zeros without touching memory).  Scalar loads return out of order, so any
  // use of one waits for every outstanding scalar and LDS access; per-tile
  // scalar loads would stall every tile on the metadata of the tiles after it.
  struct Meta {
    int info, j, vf, kslot, vslot;
  };
  auto unpack = [](const int4& v) {
    Meta m;
    m.kslot = __builtin_amdgcn_readfirstlane(v.x);
    m.vslot = __builtin_amdgcn_readfirstlane(v.y);
    const int z = __builtin_amdgcn_readfirstlane(v.z);
    m.info = z & 0x1ff;
    m.vf = ((z >> 9) & 1) ? 1 : 2;
    m.j = (int)((unsigned)z >> 10);
    return m;
  };
  auto fetch = [&](int e) { return unpack(meta[min(e - first, MAX_PER)]); };
  auto k_scales = [&](int e) {
    const float4 s4 = metk[min(e - first, MAX_PER)];
    kmax = fmaxf(fmaxf(s4.x, s4.y), fmaxf(s4.z, s4.w));
    kav[0] = (lq >> 4) ? s4.y : s4.x;
    kav[1] = (lq >> 4) ? s4.w : s4.z;
  };
  // DUP layout, 4-bit keys: lane L scores key 32*half + lq itself with packed 4-bit dot products, so
  // it loads that key's 128 features: the 16 bytes at P*1024 + 16*(32*fh + lq) for P = 2*half + i/2,
  // fh = i%2 (fragments 2P and 2P+1 of the record, feature half fh)
  int k4off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) k4off[i] = (2 * half + (i >> 1)) * 1024 + 512 * (i & 1) + 16 * lq;
  auto load_k = [&](const Meta& m) {
    const int is4 = (m.info >> 8) & 1;
    // The same eight 16-byte loads for either width (a per-format load sequence
    // would make the compiler wait for every outstanding load at each tile): a
    // K8 record is fragments 0..7; a K4 record takes four loads (its fragment
    // pairs, or with DUP the lane's own key), and the upper four loads are past
    // the end of its 4 KiB record (zeros, no memory access).
    const __amdgpu_buffer_rsrc_t rk =
        is4 ? record_rsrc(a.k4c, m.kslot, a.n_k4, K4_BYTES) : record_rsrc(a.k8c, m.kslot, a.n_k8, K8_BYTES);
#pragma unroll
    for (int F = 0; F < 8; ++F) {
      const int vo = (DUP && F < 4 && is4) ? k4off[F] : L * 16 + F * 1024;
      kf[F] = __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 0, LOAD_STREAM);
    }
  };
  auto load_v = [&](const Meta& m) {
    const bool v4 = m.vf != 1;
    const __amdgpu_buffer_rsrc_t rv =
        v4 ? record_rsrc(a.v4c, m.vslot, a.n_v4, V4_BYTES) : record_rsrc(a.v8c, m.vslot, a.n_v8, V8_BYTES);
#pragma unroll
    for (int F = 0; F < 8; ++F) vf8[F] = __builtin_amdgcn_raw_buffer_load_b128(rv, L * 16 + F * 1024, 0, LOAD_STREAM);
  };
  // fragment f of a 4-bit record: half (f & 1) of load f >> 1, expanded to 16*code bytes
  auto frag4 = [](const v4i (&w)[8], int f) {
    const v4i p = w[f >> 1];
    return (f & 1) ? unpack16(v4i{p[2], p[3], 0, 0}) : unpack16(p);
  };


  // Entry first + L of the split (clamped into the entry table, so every lane
  // loads; the tile index is clamped too, as entries past the count are not
  // tiles); lanes past the split's end get the out-of-range offsets.  Either
  // source only finds the entries; the first tile's record loads and the use
  // of Q follow them.  With a task table (TASKS) that is straight-line code,
  // so the compiler waits for Q with the 16 record loads still in flight and
  // the quantization overlaps their latency (after a join of two paths it
  // waits for every outstanding load).
  int4 w = make_int4(NO_RECORD, NO_RECORD, (1 << 9), 0);  // kslot, vslot, info | v8 << 9 | j << 10
  float4 ka = make_float4(1.f, 1.f, 1.f, 1.f);
  if constexpr (TASKS) {
    // the task table holds this lane's entry ready: the records stream right away
    w = make_int4(task_w.x, task_w.y, task_w.z, 0);
    ka = task_k;
  } else {
    const bool valid = L < last - first;
    // (independent of the split's entry count, so these loads need not wait for it)
    const int64_t li = mbase + min(first + min(L, last - first - 1), a.maxn - 1);
    const int info = a.kinfo[li], er = a.entry[li], vs = a.slot[li];
    // (keep the entry and slot loads ahead of the K scales: the tile-index load below waits for
    // the entry, and waits count loads in issue order)
    __builtin_amdgcn_sched_barrier(0);
    const int is4 = valid ? (info >> 8) & 1 : 0;
    const int j = min(max(er & ENTRY_TILE, 0), a.tiles_max - 1);
    const float4 kl = *reinterpret_cast<const float4*>((is4 ? a.ka4 : a.ka) + (hb * a.tiles_max + j) * 4);
    __builtin_amdgcn_sched_barrier(0);
    // The V format: from the entry when the cache marked it there, else from fmt, one memory
    // round trip after the entry (a uniform branch: the marked path never waits for a fmt load).
    int vf = (er & ENTRY_V8) ? 1 : 2;
    if (!__builtin_amdgcn_readfirstlane((int)__all(!valid || (er & ENTRY_VFMT)))) {
      vf = a.fmt[(int64_t)b * a.tiles_max + j];
      asm volatile("" ::"v"(vf));  // wait for it here, so that no wait follows the join
    }
    if (valid) {
      w = make_int4((int)((unsigned)info >> 9), vs, (info & 0x1ff) | ((vf == 1) << 9) | (j << 10), 0);
      ka = kl;
    }
  }
  // the wave's first tile (lane wv holds entry first + wv): K and V stream while Q is quantized
  const Meta m0 = unpack(int4{__builtin_amdgcn_readlane(w.x, wv), __builtin_amdgcn_readlane(w.y, wv),
                              __builtin_amdgcn_readlane(w.z, wv), 0});
  load_k(m0);
  load_v(m0);
  Meta mc = m0;  // the current tile
  float xv[16];  // this lane's 16 Q features
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint2 raw = qraw[i];
    xv[4 * i] = bf16f(raw.x & 0xffffu);
    xv[4 * i + 1] = bf16f(raw.x >> 16);
    xv[4 * i + 2] = bf16f(raw.y & 0xffffu);
    xv[4 * i + 3] = bf16f(raw.y >> 16);
  }
  meta[L] = w;
  metk[L] = ka;
  if (L == 0) {
    meta[MAX_PER] = make_int4(NO_RECORD, NO_RECORD, (1 << 9), 0);
    metk[MAX_PER] = make_float4(1.f, 1.f, 1.f, 1.f);
  }

  // ---- in-kernel Q quantization of the g rows (common_device.cuh:291-315)
  {
    rotate128_x16(xv, qt);
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(xv[i]));
    mx = lanes8_max(mx);
    const bool live = qrw < g;
    const float inv = mx > 0.f ? 127.f / mx : 0.f, inv4 = mx > 0.f ? 7.f / mx : 0.f;
    uint32_t w8[4], w4[4], c4[16];
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      w8[wd] = 0u;
      w4[wd] = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = xv[4 * wd + i];
        w8[wd] |= ((uint32_t)(int)__builtin_rintf(x * inv) & 0xffu) << (8 * i);
        c4[4 * wd + i] = (uint32_t)(int)__builtin_rintf(x * inv4) & 0xfu;
        w4[wd] |= ((uint32_t)((((int)c4[4 * wd + i]) ^ 8) - 8) & 0xffu) << (8 * i);
      }
      if (!live) w8[wd] = w4[wd] = 0u;
    }
    *reinterpret_cast<uint4*>(&q8s[qrw][qt * 16]) = make_uint4(w8[0], w8[1], w8[2], w8[3]);
    *reinterpret_cast<uint4*>(&q4s[qrw][qt * 16]) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    // packed 4-bit words of features fb..fb+7 (fb = 16*qt, 16*qt + 8) in the nibble order of a K4
    // record word: features fb, fb+4, fb+1, fb+5, fb+2, fb+6, fb+3, fb+7
    uint32_t pw[2] = {0u, 0u};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int n = 0; n < 8; ++n) pw[h] |= c4[8 * h + (n >> 1) + 4 * (n & 1)] << (4 * n);
    *reinterpret_cast<uint2*>(&q4w[qrw][2 * qt]) = live ? make_uint2(pw[0], pw[1]) : make_uint2(0u, 0u);
    if (qt == 0) {
      qsc[qrw] = (live && mx > 0.f) ? mx / 127.f * a.sm_log2 : 1.17549435e-38f;
      qsc4[qrw] = (live && mx > 0.f) ? mx / 7.f * a.sm_log2 : 1.17549435e-38f;
    }
  }
  for (int i = L; i < MAX_GROUP * BN / 4; i += 64) reinterpret_cast<uint32_t*>(&pls[0][0])[i] = 0u;
  __syncthreads();
  // DUP: the Q operands stay in registers for the whole split.  INT8 keys: the A operand of the QK
  // MFMA (row lq is q-head lq, rows 4..7 repeat q-heads 0..3, rows 8.. zero).  INT4 keys: the packed
  // words of rows 0..R-1, in the order of the lane's four K loads (load i, word w: feature
  // 32*(2*(i/2) + w/2) + 16*(i%2) + 8*(w%2)).
  // (two waves per workgroup with 4 rows: the packed words are read from LDS at each tile instead,
  // as 64 more registers would not fit two waves per SIMD)
  constexpr bool QW_REGS = !(NW > 1 && R >= 4);
  v4i q8a[4];
  uint32_t qw[QW_REGS ? R : 1][16];
  if constexpr (DUP) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const v4i z = {0, 0, 0, 0};
      q8a[ks] = lq < MAX_GROUP ? *reinterpret_cast<const v4i*>(&q8s[lq & 3][ks * 32 + 16 * half]) : z;
    }
    if constexpr (QW_REGS) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int w = 0; w < 4; ++w) qw[r][4 * i + w] = q4w[r][4 * (2 * (i >> 1) + (w >> 1)) + 2 * (i & 1) + (w & 1)];
    }
  }
  // Q scales in registers: per row of the lane, and the owner row's
  float qsr8[R], qsr4[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    qsr8[r] = qsc[qrow(r)];
    qsr4[r] = qsc4[qrow(r)];
  }
  const float qs8_own = orow < g ? qsc[orow] : 1.17549435e-38f, qs4_own = orow < g ? qsc4[orow] : 1.17549435e-38f;
  k_scales(first + wv);
  Meta mn = fetch(first + wv + NW);
  for (int e = first + wv; e < last; e += NW) {
    const int info = mc.info;
    const int is4 = (info >> 8) & 1;
    const unsigned rowmask = info & 0xff;
    const int j = mc.j;
    const int vf = mc.vf;
    const float cur_kmax = kmax;
    // ---- S = Q K^T
    int dot[R][NK];
    if (DUP && is4) {
      // 4-bit keys: packed 4-bit dot products of the lane's key against each row (exact integers)
#pragma unroll
      for (int r = 0; r < R; ++r) dot[r][0] = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int word = 4 * (2 * (i >> 1) + (w >> 1)) + 2 * (i & 1) + (w & 1);
            const uint32_t qv = QW_REGS ? qw[QW_REGS ? r : 0][4 * i + w] : q4w[r][word];
            dot[r][0] = __builtin_amdgcn_sdot8((int)qv, kf[i][w], dot[r][0], false);
          }
    } else {
      v4i qa[4];
      if constexpr (DUP) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qa[ks] = q8a[ks];
      } else {
        const int8_t* qsrc = is4 ? &q4s[0][0] : &q8s[0][0];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          v4i z = {0, 0, 0, 0};
          // A-operand row lq is q-head lq
          qa[ks] = lq < MAX_GROUP ? *reinterpret_cast<const v4i*>(qsrc + lq * D + ks * 32 + 16 * half) : z;
        }
      }
      // with DUP rows 4..7 repeat q-heads 0..3, so the upper half of the result holds rows 0..3
      // against the second key block
      v16i s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          s[kb] = mfma_i8(qa[ks], (!DUP && is4) ? frag4(kf, kb * 4 + ks) : kf[kb * 4 + ks], s[kb]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NK; ++t) {
          const int v = DUP ? (half ? s[1][r] : s[0][r]) : s[t][r];
          dot[r][t] = (!DUP && is4) ? (v >> 4) : v;
        }
    }
    const float kv0 = kav[0], kv1 = kav[1];
    load_k(mn);  // K registers are free again (past the end: no memory access)
    k_scales(e + NW);
    float kavc[NK];
    if constexpr (DUP) kavc[0] = half ? kv1 : kv0;
    else { kavc[0] = kv0; kavc[NK - 1] = kv1; }
    bool ok[R][NK];
    float slope[R][NK], trow[R];
    // keys past the prompt exist only in its last tile; tiles after it (spilled from the tail) are full
    const int lim = j < ptiles ? prompt : INT_MAX;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int q = qrow(r);
      const bool on = q < g && ((rowmask >> q) & 1u);
      const float qs4 = qsr4[r], qs8 = qsr8[r];
      const float qs = is4 ? qs4 : qs8;
      trow[r] = -__builtin_inff();
#pragma unroll
      for (int t = 0; t < NK; ++t) {
        const int kb = DUP ? half : t;
        ok[r][t] = on && (j * BN + kb * 32 + lq < lim);
        slope[r][t] = qs * kavc[t];
        // The 16 lanes of a DPP row hold keys of one 16-key group, so one slope (>= 0): the row's
        // largest scaled score is the slope times its largest integer dot product.
        const int dm = row16_max_i(ok[r][t] ? dot[r][t] : INT_MIN);
        if (dm != INT_MIN) trow[r] = fmaxf(trow[r], slope[r][t] * (float)dm);
      }
      trow[r] = DUP ? rows_max_wave(trow[r]) : rows_max_half(trow[r], half);
    }
    // ---- per-row scalars on the owner lane (common_device.cuh:222-238)
    const float levels = vf == 1 ? 255.f : 15.f;
    float base_r[R], bq_r[R], restore_r[R];
    bool moved_any;
    float alpha = 1.f;
    {
      float tile_o = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < R; ++r) tile_o = (L & 3) == r ? trow[r] : tile_o;
      const float qs_o = is4 ? qs4_own : qs8_own;
      // Reference max: the P levels are relative to the tile's own base and bq carries 2^(base - m),
      // so m only scales acc and den alike; it moves when a tile's max exceeds it by more than 16
      // (bq <= 2^(16 + margin)), and most tiles skip the rescale.
      const float n = tile_o > m_o + 16.f ? tile_o : m_o;
      moved_any = __any(n != m_o);
      if (moved_any) alpha = texp2(m_o - n);
      m_o = n;
      const bool any = tile_o > -__builtin_inff();
      float base = any ? tile_o : n;
      base += __builtin_fmaf(qs_o * cur_kmax, 0.75f, fabsf(base) * 2.4e-7f);
      // the reference divides by the level count under fast math; here: times its reciprocal
      const float bq = any ? texp2(base - n) * (vf == 1 ? 1.f / 255.f : 1.f / 15.f) : 0.f;
      const float restore = vf == 1 ? bq : bq * (127.f / 7.f);
      // row q's scalars are in lane q (q < 4) or 32 + q - 4; every lane reads its rows' by readlane
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (DUP) {
          base_r[r] = readlane_f(base, r);
          bq_r[r] = readlane_f(bq, r);
          restore_r[r] = readlane_f(restore, r);
        } else {
          base_r[r] = half ? readlane_f(base, 32 + r) : readlane_f(base, r);
          bq_r[r] = half ? readlane_f(bq, 32 + r) : readlane_f(bq, r);
          restore_r[r] = half ? readlane_f(restore, 32 + r) : readlane_f(restore, r);
        }
      }
    }
    const float (&base)[R] = base_r, (&bq)[R] = bq_r, (&restore)[R] = restore_r;
    if (moved_any) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float al = DUP ? readlane_f(alpha, r) : (half ? readlane_f(alpha, 32 + r) : readlane_f(alpha, r));
        den[r] *= al;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[cb][r] *= al;
      }
    }
    // ---- dithered P levels (common_device.cuh:239-246), transposed through LDS
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint32_t psum = 0;
#pragma unroll
      for (int t = 0; t < NK; ++t) {
        const int kb = DUP ? half : t;
        const int d = dot[r][t];
        // both forms of the score, selected by the tile's K width (selects, no branches): the
        // 8-bit form is the reference's magic float 1.5*2^23 + d with the bias folded into c
        const float x = is4 ? (float)d : __uint_as_float(MAGIC_BITS + (uint32_t)d);
        const float c = is4 ? -base[r] : (-slope[r][t] * MAGIC) - base[r];
        const float arg = ok[r][t] ? __builtin_fmaf(slope[r][t], x, c) : -__builtin_inff();
        const uint32_t dith = 0x47400000u | (ok[r][t] ? (uint32_t)d & 0xffu : 0u);
        // texp2, not the hardware exp2: with 15 levels (INT4 V) a level that a 1-ulp difference
        // moves across a rounding boundary moves the output by up to ~4e-2 (measured), and this
        // memory-bound kernel has the VALU time for the exact exp2
        const uint32_t y = __float_as_uint(__builtin_fmaf(texp2(arg), levels, __uint_as_float(dith)));
        const uint32_t p = (y >> 8) & 0xffu;
        psum += p;
        pls[qrow(r)][kb * 32 + lq] = (uint8_t)p;
      }
      den[r] = __builtin_fmaf((float)psum, bq[r], den[r]);
    }
    if constexpr (NW == 1) {
      __syncthreads();
    } else {
      // the P levels are this wave's own: order its LDS writes before its reads
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // ---- O = P V
    v4i pa[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      v4i w = {0, 0, 0, 0};
      if (lq < MAX_GROUP) {
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) w[pp] = *reinterpret_cast<const int*>(&pls[lq][kb * 32 + 8 * pp + 4 * half]);
      }
      pa[kb] = w;
    }
    const Meta mnn = fetch(e + 2 * NW);
    if (vf == 1) {
      const v4i neg127 = {(int)0x81818181u, (int)0x81818181u, (int)0x81818181u, (int)0x81818181u};
      const v4i p0 = pa[0] ^ 0x7f7f7f7f, p1 = pa[1] ^ 0x7f7f7f7f;  // 127 - P as s8
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        v16i d = {};
        d = mfma_i8(neg127, vf8[cb * 2], d);
        d = mfma_i8(neg127, vf8[cb * 2 + 1], d);
        d = mfma_i8(p0, vf8[cb * 2], d);
        d = mfma_i8(p1, vf8[cb * 2 + 1], d);  // = -sum_k P v
#pragma unroll
        for (int r = 0; r < R; ++r) acc[cb][r] = __builtin_fmaf((float)d[r], -restore[r], acc[cb][r]);
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        v16i d = {};
        d = mfma_i8(pa[0], frag4(vf8, cb * 2), d);
        d = mfma_i8(pa[1], frag4(vf8, cb * 2 + 1), d);  // = 16 * sum_k P v
#pragma unroll
        for (int r = 0; r < R; ++r) acc[cb][r] = __builtin_fmaf((float)(d[r] >> 4), restore[r], acc[cb][r]);
      }
    }
    load_v(mn);  // V registers are free again
    mc = mn;
    mn = mnn;
  }

  // ---- split partials (common_device.cuh:355-370)

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int o = 1; o < (DUP ? 64 : 32); o <<= 1) den[r] += __shfl_xor(den[r], o, 64);
  if constexpr (NW > 1) {
    // wave 1 hands its (m, l, o) to wave 0, which rescales both to the larger m
    __shared__ float cm[2][4], cd[2][4];  // [half][r]
    __shared__ float co[4][R][64];
    if (wv == 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) co[cb][r][L] = acc[cb][r];
        if (lq == 0) cd[half][r] = den[r];
      }
      if (owner && lq < 4) cm[DUP ? 0 : half][L & 3] = m_o;
    }
    __syncthreads();
    if (wv == 1) return;
    float m_new = m_o;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int hh = DUP ? 0 : half;
      const float m0 = DUP ? readlane_f(m_o, r) : (half ? readlane_f(m_o, 32 + r) : readlane_f(m_o, r));
      const float m1 = cm[hh][r];
      const float mx = fmaxf(m0, m1), a0 = texp2(m0 - mx), a1 = texp2(m1 - mx);
      den[r] = __builtin_fmaf(cd[half][r], a1, den[r] * a0);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) acc[cb][r] = __builtin_fmaf(co[cb][r][L], a1, acc[cb][r] * a0);
      if ((L & 3) == r) m_new = mx;
    }
    m_o = m_new;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int q = 4 * half + r;
    if (q < g) {
      const int64_t idx = ((int64_t)b * a.hq + kh * g + q) * a.splits + split;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) a.po[idx * D + cb * 32 + lq] = acc[cb][r];
      if (lq == 0) a.pl[idx] = den[r];
    }
  }
  if (owner && lq < 4 && orow < g) a.pm[((int64_t)b * a.hq + kh * g + orow) * a.splits + split] = m_o;
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
  const int64_t* tail_base;  // tokens moved from the tail into the cache since the store (may be null: 0)
  void* out;             // [B][Hq][1][128], strides osb, osh
  int out_dtype;         // 0 = fp32, 1 = bf16
  int64_t qsb, qsh, tsb, tsh, tst, csb, csh, osb, osh;
  int hq, hk, splits, max_tail;
  float sm_log2;
  int wide;  // the grid has at least SHORT_WIDE workgroups per CU (the one-wave form may pay)
};

// LSE merge of the split partials with the exact bf16 tail
// (common_device.cuh:373-469).  One 256-thread workgroup per (sequence, q-head),
// XCD-aware so the q-heads of one KV head share an L2 for their tail reads.
// Every global load that does not depend on another is issued first (the split
// partials of up to 16 splits, the first 32 tail tokens' K rows and first 64
// tail tokens' V rows), so a short tail costs one memory round trip; longer
// tails and more splits continue in loops.  Tail scores: 8 lanes per token (16
// channels each); tail values: 16 lanes per token (8 channels each).
__device__ __forceinline__ void merge_four(const MergeArgs& a) {
  __shared__ float ts[MAX_TAIL];  // tail scores
  __shared__ float vo[16][D];     // tail value sums of the 16 token groups
  __shared__ float wo[4][D];      // split sums of the four waves
  __shared__ float wred[4][2];    // per wave: max, split weight sum
  __shared__ float ltg[16];       // tail weight sums of the 16 token groups
  int hq, b;
  {
    const int total = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int q8 = total >> 3, r8 = total & 7, x = lin & 7;
    const int w = x * q8 + min(x, r8) + (lin >> 3);
    hq = w % gridDim.x;
    b = w / gridDim.x;
  }
  const int g = a.hq / a.hk, kh = hq / g;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // the tail holds step - tail_base tokens before this one (the reference: step, clamped to max_tail - 1)
  const int64_t held = *a.step - (a.tail_base != nullptr ? *a.tail_base : 0);
  const int prior = (int)max((int64_t)0, min((int64_t)a.max_tail - 1, held)), tail = prior + 1;
  const int64_t hb = (int64_t)b * a.hk + kh;
  const float* vmean = a.vstat + hb * 3 * D;
  const float* vscale = vmean + D;
  const uint16_t* kc = a.kcur + b * a.csb + kh * a.csh;
  const uint16_t* vc = a.vcur + b * a.csb + kh * a.csh;
  const uint16_t* kt = a.ktail + b * a.tsb + kh * a.tsh;
  const uint16_t* vt = a.vtail + b * a.tsb + kh * a.tsh;
  const int64_t pbase = ((int64_t)b * a.hq + hq) * a.splits;
  const int sgrp = tid >> 3, sc0 = (tid & 7) * 16;  // score layout: token group, first channel
  const int vgrp = tid >> 4, vc0 = (tid & 15) * 8;  // value layout
  // ---- loads issued up front
  float qv[16], mu[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    qv[i] = bf16f(a.q[b * a.qsb + hq * a.qsh + sc0 + i]);
    mu[i] = a.kstat[hb * 3 * D + sc0 + i];
  }
  uint4 kraw[2];
  {
    const int t = min(sgrp, tail - 1);
    const uint16_t* row = (t < prior ? kt + (int64_t)t * a.tst : kc) + sc0;
    kraw[0] = *reinterpret_cast<const uint4*>(row);
    kraw[1] = *reinterpret_cast<const uint4*>(row + 8);
  }
  uint4 vraw[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = min(vgrp + u * 16, tail - 1);
    vraw[u] = *reinterpret_cast<const uint4*>((t < prior ? vt + (int64_t)t * a.tst : vc) + vc0);
  }
  float pmv[4], plv[4];
  float2 pov[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int s = min(wave + 4 * u, a.splits - 1);
    pmv[u] = a.pm[pbase + s];
    plv[u] = a.pl[pbase + s];
    pov[u] = *reinterpret_cast<const float2*>(a.po + (pbase + s) * D + lane * 2);
  }
  const float vmv = tid < D ? vmean[tid] : 0.f, vsv = tid < D ? vscale[tid] : 0.f;
  if (hq % g == 0 && tid < D) {
    a.ktail[b * a.tsb + kh * a.tsh + prior * a.tst + tid] = kc[tid];
    a.vtail[b * a.tsb + kh * a.tsh + prior * a.tst + tid] = vc[tid];
  }
  // ---- tail scores q . (k - kmean) * sm_log2
  auto score = [&](const uint4 (&raw)[2], int t) {
    const uint32_t w[8] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w, raw[1].x, raw[1].y, raw[1].z, raw[1].w};
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float kx = bf16f((uint16_t)(w[i >> 1] >> (16 * (i & 1))));
      part = __builtin_fmaf(qv[i], kx - mu[i], part);
    }
    part += lane_xor8<1>(part);
    part += lane_xor8<2>(part);
    part += lane_xor8<4>(part);
    if ((tid & 7) == 0 && t < tail) ts[t] = part * a.sm_log2;
  };
  score(kraw, sgrp);
  for (int t0 = sgrp + 32; t0 < tail; t0 += 32) {
    const int t = min(t0, tail - 1);
    const uint16_t* row = (t < prior ? kt + (int64_t)t * a.tst : kc) + sc0;
    uint4 raw[2] = {*reinterpret_cast<const uint4*>(row), *reinterpret_cast<const uint4*>(row + 8)};
    score(raw, t0);
  }
  float pm_own = -3.402823466e38f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (wave + 4 * u < a.splits) pm_own = fmaxf(pm_own, pmv[u]);
  for (int s = wave + 16; s < a.splits; s += 4) pm_own = fmaxf(pm_own, a.pm[pbase + s]);
  __syncthreads();
  float m = pm_own;
  for (int t = tid; t < tail; t += 256) m = fmaxf(m, ts[t]);
  m = wave_max(m);
  if (lane == 0) wred[wave][0] = m;
  __syncthreads();
  m = fmaxf(fmaxf(wred[0][0], wred[1][0]), fmaxf(wred[2][0], wred[3][0]));
  // split sums: wave w takes splits w, w + 4, ... in order
  float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (wave + 4 * u < a.splits) {
      const float w = texp2(pmv[u] - m);
      l = __builtin_fmaf(plv[u], w, l);
      o0 = __builtin_fmaf(pov[u].x, w, o0);
      o1 = __builtin_fmaf(pov[u].y, w, o1);
    }
  }
  for (int s = wave + 16; s < a.splits; s += 4) {
    const float w = texp2(a.pm[pbase + s] - m);
    l = __builtin_fmaf(a.pl[pbase + s], w, l);
    const float2 p = *reinterpret_cast<const float2*>(a.po + (pbase + s) * D + lane * 2);
    o0 = __builtin_fmaf(p.x, w, o0);
    o1 = __builtin_fmaf(p.y, w, o1);
  }
  if (lane == 0) wred[wave][1] = l;
  wo[wave][lane * 2] = o0;
  wo[wave][lane * 2 + 1] = o1;
  // ---- tail values: each token's weight texp2(score - m) is computed by the 16 lanes that
  // accumulate its values (no separate pass and barrier); lane 0 of the group sums the weights
  {
    float av[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float lt = 0.f;
    auto accum = [&](const uint4& raw, int t) {
      const float e = t < tail ? texp2(ts[t] - m) : 0.f;
      lt += e;
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) av[i] = __builtin_fmaf(e, bf16f((uint16_t)(w[i >> 1] >> (16 * (i & 1)))), av[i]);
    };
#pragma unroll
    for (int u = 0; u < 4; ++u) accum(vraw[u], vgrp + u * 16);
    for (int t0 = vgrp + 64; t0 < tail; t0 += 4 * 16) {
      uint4 raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = min(t0 + u * 16, tail - 1);
        raw[u] = *reinterpret_cast<const uint4*>((t < prior ? vt + (int64_t)t * a.tst : vc) + vc0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) accum(raw[u], t0 + u * 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) vo[vgrp][vc0 + i] = av[i];
    if ((tid & 15) == 0) ltg[vgrp] = lt;
  }
  __syncthreads();
  if (tid >= D) return;
  float lsum = 0.f, osum = 0.f, tsum = 0.f, vsum = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    lsum += wred[w][1];
    osum += wo[w][tid];
  }
#pragma unroll
  for (int grp = 0; grp < 16; ++grp) {
    vsum += vo[grp][tid];
    tsum += ltg[grp];
  }
  const float acc = __builtin_fmaf(osum, vsv, lsum * vmv) + vsum;
  const float r = acc / (lsum + tsum);
  if (a.out_dtype == 0) static_cast<float*>(a.out)[b * a.osb + hq * a.osh + tid] = r;
  else static_cast<uint16_t*>(a.out)[b * a.osb + hq * a.osh + tid] = f32_to_bf16(r);
}

}  // namespace tri

namespace tri {

// The merge as ONE wave per (sequence, q-head), for short tails: every load that does not depend on
// another is issued first -- the first 32 tail tokens' K rows, the first 16 tokens' V rows and the
// first 16 splits' partials -- so a short tail costs one memory round trip, no workgroup barrier is
// needed, and the work grows with the tail (longer tails and more splits continue in loops and stay
// exact, only slower than decode_merge_kernel).  The arithmetic follows the reference's merge order
// exactly (common_device.cuh:373-469): a tail score is the 32-lane butterfly sum of fma chains over 4
// channels each, here laid out on 8 lanes per token (lane j holds the chains of channels 16j..16j+15,
// the butterfly's xor-16, 8 and 4 stages are DPP exchanges between lanes j ^ 4, 2, 1 and its xor-2
// and 1 stages add in registers); the split sums run in four interleaved groups (splits w, w + 4, ...)
// added in group order; the tail tokens are then added one after another.  XCD-aware (sequence,
// q-head) mapping as decode_merge_kernel.
__device__ __forceinline__ void merge_one(const MergeArgs& a) {
  __shared__ float ts[MAX_TAIL];  // tail scores
  int hq, b;
  {
    const int total = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int q8 = total >> 3, r8 = total & 7, x = lin & 7;
    const int w = x * q8 + min(x, r8) + (lin >> 3);
    hq = w % gridDim.x;
    b = w / gridDim.x;
  }
  const int g = a.hq / a.hk, kh = hq / g;
  const int L = threadIdx.x;
  const int64_t held = *a.step - (a.tail_base != nullptr ? *a.tail_base : 0);
  const int prior = (int)max((int64_t)0, min((int64_t)a.max_tail - 1, held)), tail = prior + 1;
  const int64_t hb = (int64_t)b * a.hk + kh;
  const float* vmean = a.vstat + hb * 3 * D;
  const float* vscale = vmean + D;
  const uint16_t* kc = a.kcur + b * a.csb + kh * a.csh;
  const uint16_t* vc = a.vcur + b * a.csb + kh * a.csh;
  const uint16_t* kt = a.ktail + b * a.tsb + kh * a.tsh;
  const uint16_t* vt = a.vtail + b * a.tsb + kh * a.tsh;
  const int64_t pbase = ((int64_t)b * a.hq + hq) * a.splits;
  const int splits = a.splits;
  // score layout: token 8u + (L >> 3) in pass u, lane j = L & 7 channels 16j..16j+15; value layout:
  // channels 2L, 2L + 1
  const int tg = L >> 3, c16 = (L & 7) * 16, c2 = 2 * L;
  // ---- loads issued up front
  float qv[16], mu[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    qv[i] = bf16f(a.q[b * a.qsb + hq * a.qsh + c16 + i]);
    mu[i] = a.kstat[hb * 3 * D + c16 + i];
  }
  auto krow = [&](int t, uint4 (&raw)[2]) {
    const int tt = min(t, tail - 1);
    const uint16_t* row = (tt < prior ? kt + (int64_t)tt * a.tst : kc) + c16;
    raw[0] = *reinterpret_cast<const uint4*>(row);
    raw[1] = *reinterpret_cast<const uint4*>(row + 8);
  };
  auto vrow = [&](int t) {
    const int tt = min(t, tail - 1);
    return *reinterpret_cast<const uint32_t*>((tt < prior ? vt + (int64_t)tt * a.tst : vc) + c2);
  };
  const int npass = (tail + 7) >> 3;
  uint4 kraw[4][2];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (u < npass) krow(8 * u + tg, kraw[u]);
  uint32_t vraw[16];
#pragma unroll
  for (int t = 0; t < 16; ++t)
    if (t < tail) vraw[t] = vrow(t);
  const float pms = L < splits ? a.pm[pbase + L] : -3.402823466e38f;
  const float pls = L < splits ? a.pl[pbase + L] : 0.f;
  float2 pov[16];
#pragma unroll
  for (int u = 0; u < 16; ++u)
    if (u < splits) pov[u] = *reinterpret_cast<const float2*>(a.po + (pbase + u) * D + c2);
  const float2 vmv = *reinterpret_cast<const float2*>(vmean + c2), vsv = *reinterpret_cast<const float2*>(vscale + c2);
  if (hq % g == 0) {
    *reinterpret_cast<uint32_t*>(a.ktail + b * a.tsb + kh * a.tsh + prior * a.tst + c2) =
        *reinterpret_cast<const uint32_t*>(kc + c2);
    *reinterpret_cast<uint32_t*>(a.vtail + b * a.tsb + kh * a.tsh + prior * a.tst + c2) =
        *reinterpret_cast<const uint32_t*>(vc + c2);
  }
  // ---- tail scores q . (k - kmean) * sm_log2 (the reference's 32-lane butterfly, see above)
  auto score = [&](const uint4 (&raw)[2], int t) {
    const uint32_t w[8] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w, raw[1].x, raw[1].y, raw[1].z, raw[1].w};
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int ch = 4 * i + c;
        const float kx = bf16f((uint16_t)(w[ch >> 1] >> (16 * (ch & 1))));
        p[i] = __builtin_fmaf(qv[ch], kx - mu[ch], p[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] += lane_xor8<4>(p[i]);  // butterfly stage 16
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] += lane_xor8<2>(p[i]);  // stage 8
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] += lane_xor8<1>(p[i]);  // stage 4
    const float s = (p[0] + p[2]) + (p[1] + p[3]);          // stages 2 and 1
    if ((L & 7) == 0 && t < tail) ts[t] = s * a.sm_log2;
  };
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (u < npass) score(kraw[u], 8 * u + tg);
  for (int u = 4; u < npass; ++u) {
    uint4 raw[2];
    krow(8 * u + tg, raw);
    score(raw, 8 * u + tg);
  }
  // (one wave: its LDS accesses run in issue order, so the scores written above are seen below once
  // the compiler keeps the order; no workgroup barrier, as merge_one also runs in a four-wave
  // workgroup whose other waves have left)
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  // ---- reference max over the splits and the tail
  float m = pms;
  for (int sp = 64 + L; sp < splits; sp += 64) m = fmaxf(m, a.pm[pbase + sp]);
  for (int t = L; t < tail; t += 64) m = fmaxf(m, ts[t]);
  m = wave_max(m);
  // ---- split sums: group w holds splits w, w + 4, ... in order; the groups are added in order
  auto split_m = [&](int sp) {
    return sp < 64 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pms), sp)) : a.pm[pbase + sp];
  };
  auto split_l = [&](int sp) {
    return sp < 64 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pls), sp)) : a.pl[pbase + sp];
  };
  float total = 0.f, acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float wl = 0.f, wo0 = 0.f, wo1 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int sp = w + 4 * k;
      if (sp < splits) {
        const float wt = texp2(split_m(sp) - m);
        wl = __builtin_fmaf(split_l(sp), wt, wl);
        wo0 = __builtin_fmaf(pov[sp].x, wt, wo0);
        wo1 = __builtin_fmaf(pov[sp].y, wt, wo1);
      }
    }
    for (int sp = w + 16; sp < splits; sp += 4) {
      const float wt = texp2(split_m(sp) - m);
      wl = __builtin_fmaf(split_l(sp), wt, wl);
      const float2 p = *reinterpret_cast<const float2*>(a.po + (pbase + sp) * D + c2);
      wo0 = __builtin_fmaf(p.x, wt, wo0);
      wo1 = __builtin_fmaf(p.y, wt, wo1);
    }
    total += wl;
    acc0 += wo0;
    acc1 += wo1;
  }
  acc0 = __builtin_fmaf(acc0, vsv.x, total * vmv.x);
  acc1 = __builtin_fmaf(acc1, vsv.y, total * vmv.y);
  // ---- tail values, one token after another (lane t holds token t's weight for t < 64)
  const float e_own = L < tail ? texp2(ts[L] - m) : 0.f;
  auto add = [&](float e, uint32_t raw) {
    total += e;
    acc0 = __builtin_fmaf(e, bf16f((uint16_t)(raw & 0xffffu)), acc0);
    acc1 = __builtin_fmaf(e, bf16f((uint16_t)(raw >> 16)), acc1);
  };
  auto weight = [&](int t) {
    return t < 64 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e_own), t)) : texp2(ts[t] - m);
  };
#pragma unroll
  for (int t = 0; t < 16; ++t)
    if (t < tail) add(weight(t), vraw[t]);
  for (int t0 = 16; t0 < tail; t0 += 16) {
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) raw[i] = vrow(t0 + i);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (t0 + i < tail) add(weight(t0 + i), raw[i]);
  }
  const float r0 = acc0 / total, r1 = acc1 / total;
  // (element stores: the output rows carry no alignment contract)
  const int64_t o = b * a.osb + hq * a.osh + c2;
  if (a.out_dtype == 0) {
    static_cast<float*>(a.out)[o] = r0;
    static_cast<float*>(a.out)[o + 1] = r1;
  } else {
    static_cast<uint16_t*>(a.out)[o] = f32_to_bf16(r0);
    static_cast<uint16_t*>(a.out)[o + 1] = f32_to_bf16(r1);
  }
}

// Tokens the merge reads from the tail: the step's own token and those before it (the reference:
// step, clamped to max_tail - 1); with tail growth the tail holds step - tail_base tokens.
__device__ __forceinline__ int merge_tail(const MergeArgs& a) {
  const int64_t held = *a.step - (a.tail_base != nullptr ? *a.tail_base : 0);
  return (int)max((int64_t)0, min((int64_t)a.max_tail - 1, held)) + 1;
}

// The merge with the form chosen on the device: one wave (merge_one, the reference's order) while
// the tail holds at most SHORT_TAIL tokens on a grid of at least SHORT_WIDE workgroups per CU (a.wide),
// four waves (merge_four) otherwise.  Measured (kernel durations, Hq 28): on 896 workgroups the one-wave
// form takes 5.5 / 6.1 / 7.6 / 10.7 us at tails of 4 / 16 / 32 / 64 tokens against 6.8 / 6.8 / 6.8 / 7.6
// for four waves; on 448 or fewer four waves are as fast or faster at every tail (4.3-5.5 us).  A
// captured graph replays one launch at steps whose tails grow, so the choice cannot be the host's:
// made here (and by the host's eager choice with the same rule), every step of an eager run and of a
// replay takes the same form and gives the same bits.  With the one-wave form the other three waves
// leave at once (merge_one has no workgroup barrier).
constexpr int SHORT_TAIL = 16;
__global__ __launch_bounds__(256) void decode_merge_kernel(MergeArgs a) {
  if (a.wide && merge_tail(a) <= SHORT_TAIL) {
    if (threadIdx.x >= 64) return;
    merge_one(a);
  } else {
    merge_four(a);
  }
}

// The one-wave form alone, whatever the tail (tri_decode_short_tail).
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void decode_merge1_kernel(MergeArgs a) {
  merge_one(a);
}

}  // namespace tri
