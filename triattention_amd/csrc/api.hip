// extern "C" entry points: argument validation, launch geometry, error text.
// One translation unit holds every kernel of the library.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <numeric>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include <hip/hip_ext.h>

#include "../../include/triattention_amd.h"
#include "cache.hip"
#include "decode.hip"
#include "prefill.hip"
#include "probe.hip"
#include "quantize.hip"
#include "tail.hip"

namespace {

thread_local std::string g_error;
// tri_attention's launch form: 0 by launch size, 1 two-wave workgroups, 2 four-wave (split key tiles)
static std::atomic<int> g_prefill_pairs{0};

int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return 1;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace

// Quantized-head decode launch with NW waves per workgroup; groups of up to 4
// q-heads use the DUP lane layout (both wave halves on rows 0..3).
// With events, the launch goes through hipExtLaunchKernel, which records them as the kernel's
// own start and stop.
template <int NW, typename K>
static void launch_one(K kernel, dim3 grid, const tri::DecodeArgs& d, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  if (e0 || e1) hipExtLaunchKernelGGL(kernel, grid, dim3(64 * NW), 0, s, e0, e1, 0, d);
  else kernel<<<grid, 64 * NW, 0, s>>>(d);
}
template <int NW, bool T>
static void launch_decode(int g, dim3 grid, const tri::DecodeArgs& d, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  switch (g) {
    case 1: launch_one<NW>(tri::decode_kernel<1, false, true, NW, 2, T>, grid, d, s, e0, e1); break;
    case 2: launch_one<NW>(tri::decode_kernel<2, false, true, NW, 2, T>, grid, d, s, e0, e1); break;
    case 3: launch_one<NW>(tri::decode_kernel<3, false, true, NW, 2, T>, grid, d, s, e0, e1); break;
    case 4: launch_one<NW>(tri::decode_kernel<4, false, true, NW, 2, T>, grid, d, s, e0, e1); break;
    default: launch_one<NW>(tri::decode_kernel<4, false, false, NW, 2, T>, grid, d, s, e0, e1); break;
  }
}

// CU count of the current device, cached per device (devices 0..63)
static int device_cus(int* cus) {
  static std::atomic<int> cached[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  const bool cacheable = e == hipSuccess && dev >= 0 && dev < 64;
  if (cacheable && cached[dev].load(std::memory_order_relaxed) > 0) {
    *cus = cached[dev].load(std::memory_order_relaxed);
    return 0;
  }
  if (e == hipSuccess) e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail("device_cus: %s", hipGetErrorString(e));
  if (cacheable) cached[dev].store(*cus, std::memory_order_relaxed);
  return 0;
}

extern "C" {

const char* tri_last_error(void) { return g_error.c_str(); }

int tri_prepare_qk(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb,
                   int64_t k_sh, int64_t k_st, int batch, int hq, int hk, int t, void* q8, float* qa, void* kp,
                   float* ka, float* partial, float* kstat, void* q4, float* qa4, void* k4p, float* ka4,
                   void* k4x, void* stream) {
  g_error.clear();
  if (!q || !k || !q8 || !qa || !kp || !ka || !partial || !kstat) return fail("prepare_qk: null buffer");
  if (batch < 1 || hq < 1 || hk < 1 || t < 1) return fail("prepare_qk: empty shape");
  if (hq % hk != 0) return fail("prepare_qk: q heads (%d) not a multiple of kv heads (%d)", hq, hk);
  const bool int4 = q4 != nullptr;
  if (int4 != (qa4 != nullptr) || int4 != (k4p != nullptr) || int4 != (ka4 != nullptr))
    return fail("prepare_qk: INT4 Q/K buffers (all or none)");
  if (!aligned(q, 8) || !aligned(k, 8) || (q_st | q_sh | q_sb | k_st | k_sh | k_sb) % 4 != 0)
    return fail("prepare_qk: Q/K rows must be 8-byte aligned");
  if (!aligned(kp, 16) || !aligned(q8, 16) || (int4 && (!aligned(k4p, 16) || !aligned(q4, 4))))
    return fail("prepare_qk: output buffers must be 16-byte aligned");
  if (k4x && (!int4 || !aligned(k4x, 16))) return fail("prepare_qk: expanded K4 records need the INT4 buffers, 16-byte aligned");
  const int tiles = (t + tri::BN - 1) / tri::BN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  tri::quantize_q_kernel<<<dim3((t + 31) / 32, hq, batch), 256, 0, s>>>(
      static_cast<const uint16_t*>(q), q_sb, q_sh, q_st, hq, t, static_cast<int8_t*>(q8), qa,
      static_cast<uint8_t*>(q4), qa4);
  tri::partial_kernel<<<dim3(tri::STAT_BLOCKS, hk, batch), tri::D / 2, 0, s>>>(static_cast<const uint16_t*>(k), k_sb,
                                                                          k_sh, k_st, hk, t, partial);
  tri::finalize_kernel<<<dim3(hk, batch), tri::D, 0, s>>>(partial, kstat, hk, t, 0);
  tri::quantize_k_kernel<<<dim3(tiles, hk, batch), 256, 0, s>>>(static_cast<const uint16_t*>(k), k_sb, k_sh, k_st,
                                                                kstat, hk, t, static_cast<uint8_t*>(kp), ka,
                                                                static_cast<uint8_t*>(k4p), ka4,
                                                                static_cast<uint8_t*>(k4x));
  return check_launch("prepare_qk");
}

int tri_pack_v(const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int batch, int hk, int t, float* partial,
               float* vstat, void* v16p, void* v8p, void* v4p, int32_t* v8sum, void* stream) {
  g_error.clear();
  if (!v || !partial || !vstat) return fail("pack_v: null buffer");
  if (batch < 1 || hk < 1 || t < 1) return fail("pack_v: empty shape");
  if (!aligned(v, 8) || (v_st | v_sh | v_sb) % 4 != 0) return fail("pack_v: V rows must be 8-byte aligned");
  if ((v16p && !aligned(v16p, 16)) || (v8p && !aligned(v8p, 16)) || (v4p && !aligned(v4p, 8)))
    return fail("pack_v: record buffers must be 16-byte aligned");
  if (v8sum && (!v8p || !aligned(v8sum, 16))) return fail("pack_v: V8 sums need the V8 records, 16-byte aligned");
  const int tiles = (t + tri::BN - 1) / tri::BN;
  const bool identity = v8p == nullptr && v4p == nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!identity)
    tri::partial_kernel<<<dim3(tri::STAT_BLOCKS, hk, batch), tri::D / 2, 0, s>>>(static_cast<const uint16_t*>(v), v_sb,
                                                                            v_sh, v_st, hk, t, partial);
  tri::finalize_kernel<<<dim3(hk, batch), tri::D, 0, s>>>(partial, vstat, hk, t, identity ? 1 : 0);
  tri::pack_v_kernel<<<dim3(tiles, hk, batch), 256, 0, s>>>(static_cast<const uint16_t*>(v), v_sb, v_sh, v_st, vstat,
                                                            hk, t, static_cast<uint8_t*>(v16p),
                                                            static_cast<uint8_t*>(v8p), static_cast<uint8_t*>(v4p),
                                                            v8sum);
  return check_launch("pack_v");
}

int tri_attention(const int32_t* order, int n_order, const int32_t* bands, int batch, int hq, int hk, int t,
                  const void* v16p, const void* v8p, const float* vstat, const void* q8, const void* k8p,
                  const float* qa8, const float* ka8, const void* q4, const void* k4p, const float* qa4,
                  const float* ka4, void* out, int out_dtype, int64_t o_sb, int64_t o_sh, int64_t o_st,
                  double scale, const int32_t* exact, const void* qr, int64_t q_sb, int64_t q_sh, int64_t q_st,
                  const void* kx, const void* vx, int nx, const int32_t* v8sum, const void* k4x, void* stream) {
  g_error.clear();
  const int tiles = (t + tri::BN - 1) / tri::BN;
  if (!order || !bands || !v16p || !vstat || !q8 || !k8p || !qa8 || !ka8 || !out)
    return fail("attention: null buffer");
  if (batch < 1 || hq < 1 || hk < 1 || t < 1) return fail("attention: empty shape");
  if (tiles > tri::MAX_TILES) return fail("attention: at most 131072 tokens");
  if (hq % hk != 0) return fail("attention: q heads not a multiple of kv heads");
  if (n_order != hq * tiles) return fail("attention: CTA order must have hq*tiles entries");
  const bool int4 = q4 != nullptr;
  if (int4 != (k4p != nullptr) || int4 != (qa4 != nullptr) || int4 != (ka4 != nullptr))
    return fail("attention: INT4 Q/K operands (all or none)");
  if (out_dtype < 0 || out_dtype > 2) return fail("attention: out dtype must be fp32, bf16 or fp16");
  if (!aligned(out, 16) || (o_st % 4) || (o_sh % 4) || (o_sb % 4))
    return fail("attention: output [B,Hq,T,128] must be 16-byte aligned with strides a multiple of 4");
  // records and per-tile K scales are copied to LDS in 16-byte pieces
  if (!aligned(v16p, 16) || !aligned(k8p, 16) || !aligned(ka8, 16) || (v8p && !aligned(v8p, 16)) ||
      (int4 && (!aligned(k4p, 16) || !aligned(ka4, 16))))
    return fail("attention: record and K-scale buffers must be 16-byte aligned");
  if (int4 && v8p == nullptr) return fail("attention: INT4 key tiles need the INT8 V records");
  if (v8sum && (!v8p || !aligned(v8sum, 16))) return fail("attention: V8 sums need the V8 records, 16-byte aligned");
  if (k4x && (!int4 || !aligned(k4x, 16)))
    return fail("attention: expanded K4 records need the INT4 operands, 16-byte aligned");
  if (exact != nullptr && (!qr || !aligned(qr, 16) || (q_sb | q_sh | q_st) % 8 != 0))
    return fail("attention: exact heads need 16-byte aligned bf16 q rows");
  if (exact != nullptr && (nx < 1 || nx > hk || !kx || !vx || !aligned(kx, 16) || !aligned(vx, 16)))
    return fail("attention: exact heads need 16-byte aligned KX/VX records of 1..hk KV heads");
  tri::PrefillArgs a;
  a.exact = exact;
  a.qr = static_cast<const uint16_t*>(qr);
  a.qsb = q_sb;
  a.qsh = q_sh;
  a.qst = q_st;
  a.kx = static_cast<const uint8_t*>(kx);
  a.vx = static_cast<const uint8_t*>(vx);
  a.nx = nx;
  a.order = order;
  a.bands = bands;
  a.v16 = static_cast<const uint8_t*>(v16p);
  a.v8 = static_cast<const uint8_t*>(v8p);
  a.vstat = vstat;
  a.q8 = static_cast<const int8_t*>(q8);
  a.k8 = static_cast<const uint8_t*>(k8p);
  a.qa = qa8;
  a.ka = ka8;
  a.q4 = static_cast<const uint8_t*>(q4);
  a.k4 = static_cast<const uint8_t*>(k4p);
  a.qa4 = qa4;
  a.ka4 = ka4;
  a.out = out;
  a.out_dtype = out_dtype;
  a.osb = o_sb;
  a.osh = o_sh;
  a.ost = o_st;
  a.hq = hq;
  a.hk = hk;
  a.t = t;
  a.sm_log2 = (float)(scale * 1.4426950408889634);
  a.v8s = v8sum;
  a.k4x = static_cast<const uint8_t*>(k4x);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Launches of at most two workgroups per CU (short prompts) leave SIMDs without a wave: each
  // workgroup then takes four waves, two pairs that split its key tiles (prefill_kernel<., 2>).
  const int pmode = g_prefill_pairs.load();
  bool pairs = pmode == 2;
  if (pmode == 0) {
    int cus = 0;
    if (device_cus(&cus) != 0) return 1;
    pairs = (int64_t)n_order * batch <= 2 * (int64_t)cus;
  }
  const dim3 grid(n_order, batch);
  if (pairs) {
    if (v8sum) tri::prefill_kernel<true, 2><<<grid, 256, 0, s>>>(a);
    else tri::prefill_kernel<false, 2><<<grid, 256, 0, s>>>(a);
  } else {
    if (v8sum) tri::prefill_kernel<true, 1><<<grid, 128, 0, s>>>(a);
    else tri::prefill_kernel<false, 1><<<grid, 128, 0, s>>>(a);
  }
  return check_launch("attention");
}

int tri_pack_exact(const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb,
                   int64_t v_sh, int64_t v_st, int batch, int hq, int hk, int t, const int32_t* exact, int nx,
                   void* kx, void* vx, void* stream) {
  g_error.clear();
  const int tiles = (t + tri::BN - 1) / tri::BN;
  if (!k || !v || !exact || !kx || !vx) return fail("pack_exact: null buffer");
  if (batch < 1 || hq < 1 || hk < 1 || t < 1) return fail("pack_exact: empty shape");
  if (tiles > tri::MAX_TILES) return fail("pack_exact: at most 131072 tokens");
  if (hq % hk != 0) return fail("pack_exact: q heads not a multiple of kv heads");
  if (nx < 1 || nx > hk) return fail("pack_exact: nx must be in [1, hk]");
  if (!aligned(k, 16) || !aligned(v, 16) || (k_sb | k_sh | k_st | v_sb | v_sh | v_st) % 8 != 0)
    return fail("pack_exact: K/V rows must be 16-byte aligned");
  if (!aligned(kx, 16) || !aligned(vx, 16)) return fail("pack_exact: KX/VX records must be 16-byte aligned");
  tri::ExactPackArgs a;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.ksb = k_sb;
  a.ksh = k_sh;
  a.kst = k_st;
  a.vsb = v_sb;
  a.vsh = v_sh;
  a.vst = v_st;
  a.exact = exact;
  a.kx = static_cast<uint8_t*>(kx);
  a.vx = static_cast<uint8_t*>(vx);
  a.hq = hq;
  a.hk = hk;
  a.t = t;
  a.nx = nx;
  tri::pack_exact_kernel<<<dim3(tiles, hk, batch), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("pack_exact");
}

static int decode_impl(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c, const float* ka,
                       const float* ka4, const int32_t* entry, const int32_t* kinfo, const int32_t* count,
                       const int32_t* fmt, const int32_t* slot, const void* v8c, const void* v4c, const float* vstat,
                       const float* kstat, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh, int64_t t_st,
                       int max_tail, const void* kcur, const void* vcur, int64_t c_sb, int64_t c_sh,
                       const int64_t* step, void* out, int out_dtype, int64_t o_sb, int64_t o_sh, float* pm, float* pl,
                       float* po, const int32_t* prompt, int batch, int hq, int hk, int maxn, int per, int tiles_max,
                       int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4, const int32_t* xslot,
                       const void* kxc, const void* vxc, int64_t n_kx, const int32_t* bounds, int nsplit,
                       const void* tasks, int n_tasks, const int64_t* tail_base, double scale, void* stream, int phase,
                       hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr) {
  g_error.clear();
  if (!q || !k8c || !ka || !entry || !kinfo || !count || !fmt || !slot || !v8c || !v4c || !vstat || !kstat ||
      !ktail || !vtail || !kcur || !vcur || !step || !out || !pm || !pl || !po || !prompt)
    return fail("decode: null buffer");
  if (batch < 1 || hq < 1 || hk < 1 || maxn < 1 || tiles_max < 1) return fail("decode: empty shape");
  if (!bounds && (per < 1 || per > tri::MAX_PER)) return fail("decode: per (tiles per split) must be in [1, 64]");
  if (bounds && (nsplit < 1 || nsplit > 65535)) return fail("decode: nsplit must be in [1, 65535] with a partition");
  if (hq % hk != 0 || hq / hk > tri::MAX_GROUP) return fail("decode: GQA group must divide and be <= 8");
  if (max_tail < 1 || max_tail > tri::MAX_TAIL) return fail("decode: max_tail must be in [1, 1024]");
  if ((k4c == nullptr) != (ka4 == nullptr)) return fail("decode: INT4 K records and scales (all or none)");
  if (out_dtype != 0 && out_dtype != 1) return fail("decode: out dtype must be fp32 or bf16");
  if (!aligned(q, 8) || (q_sh % 4) || (q_sb % 4)) return fail("decode: q rows must be 8-byte aligned");
  if (!aligned(kcur, 16) || !aligned(vcur, 16) || (c_sb % 8) || (c_sh % 8))
    return fail("decode: k/v of the new token must be 16-byte aligned rows");
  if (!aligned(ktail, 16) || !aligned(vtail, 16) || (t_sb % 8) || (t_sh % 8) || (t_st % 8))
    return fail("decode: tail buffers must be 16-byte aligned rows");
  if (!aligned(po, 16)) return fail("decode: po must be 16-byte aligned");
  const int splits = bounds ? nsplit : std::max(1, (maxn + per - 1) / per);
  // record slots: K slots in the 23-bit kinfo field, V and exact-record slots in int32
  const int64_t kslots = (int64_t)1 << 23, slots = ((int64_t)1 << 31) - 1;
  if (n_k8 < 1 || n_v8 < 1 || n_v4 < 1 || n_k8 > kslots || n_k4 > kslots || n_v8 > slots || n_v4 > slots ||
      (k4c != nullptr && n_k4 < 1))
    return fail("decode: compacted record arrays must be non-empty, K arrays of at most 2^23 records");
  if (xslot != nullptr && (!kxc || !vxc || n_kx < 1 || n_kx > slots || !aligned(kxc, 16) || !aligned(vxc, 16)))
    return fail("decode: exact heads need 16-byte aligned KX/VX record arrays, non-empty");
  tri::DecodeArgs d;
  d.xslot = xslot;
  d.kxc = static_cast<const uint8_t*>(kxc);
  d.vxc = static_cast<const uint8_t*>(vxc);
  d.n_kx = xslot ? n_kx : 0;
  d.kstat = kstat;
  d.vstat = vstat;
  d.q = static_cast<const uint16_t*>(q);
  d.k8c = static_cast<const uint8_t*>(k8c);
  d.k4c = static_cast<const uint8_t*>(k4c);
  d.ka = ka;
  d.ka4 = ka4;
  d.entry = entry;
  d.kinfo = kinfo;
  d.count = count;
  d.fmt = fmt;
  d.slot = slot;
  d.v8c = static_cast<const uint8_t*>(v8c);
  d.v4c = static_cast<const uint8_t*>(v4c);
  d.prompt = prompt;
  d.pm = pm;
  d.pl = pl;
  d.po = po;
  d.qsb = q_sb;
  d.qsh = q_sh;
  d.hq = hq;
  d.hk = hk;
  d.maxn = maxn;
  d.per = per;
  d.bounds = bounds;
  // a task table lists the splits to run (exact heads gather their splits themselves)
  d.tasks = xslot == nullptr ? static_cast<const int32_t*>(tasks) : nullptr;
  if (d.tasks && (n_tasks < 1 || !aligned(tasks, 16))) return fail("decode: a task table needs n_tasks >= 1, 16-byte aligned");
  d.tiles_max = tiles_max;
  d.splits = splits;
  d.total = (int64_t)splits * hk * batch;
  {
    // Work scatter (workgroup lin takes item lin * scatter mod launched; the XCD is lin % 8).
    // - Affine (launched = items, scatter a prime not dividing it): with items % 8 == 0 the XCD fixes
    //   w % 8, and so the split index mod gcd(splits, 8).  Harmless when every split costs about the
    //   same (a cost-balanced partition, or an odd split count, which spreads each split index over
    //   the heads), and measured ~2% faster there than the golden-ratio scatter.
    // - Golden ratio for the uniform split with an even split count: in a ragged batch a split's cost
    //   falls with its index, and the affine scatter would load one XCD 2.4x the mean (C3 in runs of
    //   32 tiles: 253 -> 123 us).  An odd launch count L (one padding item), and a multiplier whose
    //   XCD step 8 * scatter mod L is the integer nearest 0.618 L coprime with L.
    const int64_t all = (int64_t)splits * hk * batch;
    if (all >= ((int64_t)1 << 31) - 1) return fail("decode: too many splits x heads x sequences");
    if (d.tasks && n_tasks > all) return fail("decode: the task table lists more splits than exist");
    const int64_t items = d.tasks ? n_tasks : all;
    const bool pinned = bounds == nullptr && items % 8 == 0 && splits % 2 == 0;
    if (d.tasks) {
      // a task table lists its splits in the order to run them (costliest first): workgroup lin takes
      // row lin, and the XCDs receive the rows round-robin
      d.scatter = 1;
      d.launched = (int)items;
    } else if (!pinned) {
      const int primes[3] = {1000003, 1000033, 1000037};
      d.scatter = primes[0];
      for (int p : primes)
        if (items % p != 0) {
          d.scatter = p;
          break;
        }
      d.launched = (int)items;
    } else {
      const int64_t launched = items | 1;
      int64_t step = std::max<int64_t>(1, (int64_t)std::llround(0.6180339887498949 * (double)launched));
      while (std::gcd(step, launched) != 1) ++step;
      const int64_t inv2 = (launched + 1) / 2;                          // 2^-1 mod L (L odd)
      const int64_t inv8 = (inv2 * inv2 % launched) * inv2 % launched;  // 8^-1 mod L
      d.scatter = launched > 1 ? step % launched * inv8 % launched : 0;
      d.launched = (int)launched;
    }
    d.items = (int)items;
  }
  d.sm_log2 = (float)(scale * 1.4426950408889634);
  d.n_k8 = n_k8;
  d.n_k4 = k4c ? n_k4 : 0;
  d.n_v8 = n_v8;
  d.n_v4 = n_v4;
  tri::MergeArgs mg;
  mg.pm = pm;
  mg.pl = pl;
  mg.po = po;
  mg.vstat = vstat;
  mg.kstat = kstat;
  mg.q = static_cast<const uint16_t*>(q);
  mg.ktail = static_cast<uint16_t*>(ktail);
  mg.vtail = static_cast<uint16_t*>(vtail);
  mg.kcur = static_cast<const uint16_t*>(kcur);
  mg.vcur = static_cast<const uint16_t*>(vcur);
  mg.step = step;
  mg.tail_base = tail_base;
  mg.out = out;
  mg.out_dtype = out_dtype;
  mg.qsb = q_sb;
  mg.qsh = q_sh;
  mg.tsb = t_sb;
  mg.tsh = t_sh;
  mg.tst = t_st;
  mg.csb = c_sb;
  mg.csh = c_sh;
  mg.osb = o_sb;
  mg.osh = o_sh;
  mg.hq = hq;
  mg.hk = hk;
  mg.splits = splits;
  mg.max_tail = max_tail;
  mg.sm_log2 = d.sm_log2;
  {
    // the one-wave merge form pays on grids of at least SHORT_WIDE (sequence, q-head) workgroups per CU
    // (the rule DecodeCache.short_tail mirrors for its eager launches)
    int cus = 0;
    if (device_cus(&cus) != 0) return 1;
    mg.wide = (int64_t)batch * hq >= (int64_t)tri::SHORT_WIDE * cus ? 1 : 0;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (phase & 1) {
    const dim3 grid(d.launched);
    const int g = hq / hk;
    if (xslot == nullptr) {
      // One wave per workgroup while the grid fits the resident waves (two per SIMD, 8
      // workgroups per CU): each wave streams a split of its own (C1, 1,024 splits: 37.4 us,
      // against 39.3 us with two waves per workgroup; C3, 1,785 splits: 99.0-100.0 us against
      // 101.5-102.7 us, same box).  Larger grids run two waves per workgroup (alternate tiles of
      // a split), which interleave their dependency chains while the dispatcher queues the rest.
      int cus = 0;
      if (device_cus(&cus) != 0) return 1;
      const bool two = (int64_t)d.items > 8 * (int64_t)cus;
      if (d.tasks) {
        if (two) launch_decode<2, true>(g, grid, d, s, ev_start, ev_stop);
        else launch_decode<1, true>(g, grid, d, s, ev_start, ev_stop);
      } else {
        if (two) launch_decode<2, false>(g, grid, d, s, ev_start, ev_stop);
        else launch_decode<1, false>(g, grid, d, s, ev_start, ev_stop);
      }
    } else {
      // groups of up to 4 q-heads use the DUP lane layout (both wave halves on rows 0..3)
      switch (g) {
        case 1: launch_one<1>(tri::decode_kernel<1, true, true>, grid, d, s, ev_start, ev_stop); break;
        case 2: launch_one<1>(tri::decode_kernel<2, true, true>, grid, d, s, ev_start, ev_stop); break;
        case 3: launch_one<1>(tri::decode_kernel<3, true, true>, grid, d, s, ev_start, ev_stop); break;
        case 4: launch_one<1>(tri::decode_kernel<4, true, true>, grid, d, s, ev_start, ev_stop); break;
        default: launch_one<1>(tri::decode_kernel<4, true, false>, grid, d, s, ev_start, ev_stop); break;
      }
    }
  }
  if (phase & 2) {
    // phase bit 4: the merge as one wave per (sequence, q-head), for short tails
    if (phase & 4) tri::decode_merge1_kernel<<<dim3(hq, batch), 64, 0, s>>>(mg);
    else tri::decode_merge_kernel<<<dim3(hq, batch), 256, 0, s>>>(mg);
  }
  return check_launch("decode");
}

// ---- decode without allocation (tri_decode_noalloc)
// The split partials pm, pl, po of one call live in this file-scope device array: one copy per GPU,
// held until the process ends.  Host code never passes `scratch` itself (its host-side name is not a
// device address); it passes the address hipGetSymbolAddress returns, taken once per device.
constexpr int64_t NOALLOC_FLOATS = (int64_t)24 << 18;  // 24 MiB of fp32
static __device__ __align__(256) float scratch[NOALLOC_FLOATS];

// Per device: the scratch address, and the stream and completion event of the last call that used the
// scratch.  A call on another stream while that event is pending would overwrite partials the earlier
// call's kernels still read, so it is refused; calls on one stream are ordered by the stream itself.
struct NoallocDevice {
  float* ptr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t stream = nullptr;
  bool used = false;
};
static std::mutex g_noalloc_mu;
static NoallocDevice g_noalloc[64];

// Set-up on the first call on a device (that device current): the scratch array's address and one event.
static int noalloc_device(NoallocDevice** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail("decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail("decode_noalloc: device %d beyond the 64 this library tracks", dev);
  NoallocDevice& d = g_noalloc[dev];
  if (d.ptr == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail("decode_noalloc: hipGetSymbolAddress of the scratch array: %s", hipGetErrorString(e));
    e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
    if (e != hipSuccess) return fail("decode_noalloc: hipEventCreateWithFlags: %s", hipGetErrorString(e));
    d.ptr = static_cast<float*>(p);
  }
  *out = &d;
  return 0;
}

#define TRI_DECODE_ARGS                                                                                      \
  q, q_sb, q_sh, k8c, k4c, ka, ka4, entry, kinfo, count, fmt, slot, v8c, v4c, vstat, kstat, ktail, vtail, t_sb, t_sh, \
      t_st, max_tail, kcur, vcur, c_sb, c_sh, step, out, out_dtype, o_sb, o_sh, pm, pl, po, prompt, batch, hq, hk,  \
      maxn, per, tiles_max, n_k8, n_k4, n_v8, n_v4, xslot, kxc, vxc, n_kx, bounds, nsplit, tasks, n_tasks,          \
      tail_base, scale, stream
#define TRI_DECODE_PARAMS                                                                                          \
  const void *q, int64_t q_sb, int64_t q_sh, const void *k8c, const void *k4c, const float *ka, const float *ka4,  \
      const int32_t *entry, const int32_t *kinfo, const int32_t *count, const int32_t *fmt, const int32_t *slot,  \
      const void *v8c, const void *v4c, const float *vstat, const float *kstat, void *ktail, void *vtail,          \
      int64_t t_sb, int64_t t_sh, int64_t t_st, int max_tail, const void *kcur, const void *vcur, int64_t c_sb,    \
      int64_t c_sh, const int64_t *step, void *out, int out_dtype, int64_t o_sb, int64_t o_sh, float *pm,          \
      float *pl, float *po, const int32_t *prompt, int batch, int hq, int hk, int maxn, int per, int tiles_max,    \
      int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4, const int32_t *xslot, const void *kxc,           \
      const void *vxc, int64_t n_kx, const int32_t *bounds, int nsplit, const void *tasks, int n_tasks,      \
      const int64_t *tail_base, double scale, void *stream

int tri_decode(TRI_DECODE_PARAMS) { return decode_impl(TRI_DECODE_ARGS, 3); }
int tri_decode_partials(TRI_DECODE_PARAMS) { return decode_impl(TRI_DECODE_ARGS, 1); }
int tri_decode_merge(TRI_DECODE_PARAMS) { return decode_impl(TRI_DECODE_ARGS, 2); }
int tri_decode_short_tail(TRI_DECODE_PARAMS) { return decode_impl(TRI_DECODE_ARGS, 3 | 4); }
int tri_decode_merge_short_tail(TRI_DECODE_PARAMS) { return decode_impl(TRI_DECODE_ARGS, 2 | 4); }
int tri_decode_partials_timed(TRI_DECODE_PARAMS, void* ev_start, void* ev_stop) {
  return decode_impl(TRI_DECODE_ARGS, 1, static_cast<hipEvent_t>(ev_start), static_cast<hipEvent_t>(ev_stop));
}

int tri_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c, const float* ka,
                       const float* ka4, const int32_t* entry, const int32_t* kinfo, const int32_t* count,
                       const int32_t* fmt, const int32_t* slot, const void* v8c, const void* v4c, const float* vstat,
                       const float* kstat, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh, int64_t t_st,
                       int max_tail, const void* kcur, const void* vcur, int64_t c_sb, int64_t c_sh,
                       const int64_t* step, void* out, int out_dtype, int64_t o_sb, int64_t o_sh,
                       const int32_t* prompt, int batch, int hq, int hk, int maxn, int per, int tiles_max,
                       int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4, const int32_t* xslot,
                       const void* kxc, const void* vxc, int64_t n_kx, const int32_t* bounds, int nsplit,
                       const void* tasks, int n_tasks, const int64_t* tail_base, double scale, void* stream) {
  g_error.clear();
  if (batch < 1 || hq < 1 || hk < 1 || maxn < 1) return fail("decode_noalloc: empty shape");
  if (!bounds && (per < 1 || per > tri::MAX_PER)) return fail("decode_noalloc: per (tiles per split) must be in [1, 64]");
  if (bounds && (nsplit < 1 || nsplit > 65535)) return fail("decode_noalloc: nsplit must be in [1, 65535]");
  const int64_t splits = bounds ? nsplit : std::max(1, (maxn + per - 1) / per);
  // split partials: (m, l) and o[128] each; pl and po start on 256-byte boundaries
  auto floats = [](int64_t n) { return 2 * ((n + 63) / 64 * 64) + n * tri::D; };
  const int64_t n = (int64_t)batch * hq * splits;
  const int64_t pad = (n + 63) / 64 * 64;
  if (floats(n) > NOALLOC_FLOATS) {
    int64_t most = NOALLOC_FLOATS / (tri::D + 2);
    while (floats(most + 1) <= NOALLOC_FLOATS) ++most;
    return fail("decode_noalloc: %lld split partials (batch %d x q-heads %d x splits %lld) exceed the %lld-float "
                "scratch (at most %lld); use tri_decode with caller buffers",
                (long long)n, batch, hq, (long long)splits, (long long)NOALLOC_FLOATS, (long long)most);
  }
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoallocDevice* nd = nullptr;
  if (noalloc_device(&nd) != 0) return 1;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  // (under stream capture nothing runs now, and querying or recording events is not allowed: a captured
  // call is not checked, and the caller keeps graph replays off other streams' calls)
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(hs, &cap);
  if (e != hipSuccess) return fail("decode_noalloc: hipStreamIsCapturing: %s", hipGetErrorString(e));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (!capturing && nd->used && nd->stream != hs) {
    e = hipEventQuery(nd->done);
    if (e == hipErrorNotReady)
      return fail("decode_noalloc: this GPU's scratch is still in use by a call on another stream; wait for that "
                  "stream (or call on it) before calling on this one");
    if (e != hipSuccess) return fail("decode_noalloc: hipEventQuery: %s", hipGetErrorString(e));
  }
  float* s = nd->ptr;
  float* pm = s;
  float* pl = s + pad;
  float* po = s + 2 * pad;
  if (tasks && xslot == nullptr) {
    // splits a task table leaves out are never written: the scratch (which holds whatever the last
    // call left) gets the empty partial in every slot first
    tri::fill_empty_partials_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, hs>>>(pm, pl, po, n);
  }
  const int rc = decode_impl(TRI_DECODE_ARGS, 3);
  if (rc == 0 && !capturing) {
    e = hipEventRecord(nd->done, hs);
    if (e != hipSuccess) return fail("decode_noalloc: hipEventRecord: %s", hipGetErrorString(e));
    nd->stream = hs;
    nd->used = true;
  }
  return rc;
}

int tri_decode_tasks(const float* ka, const float* ka4, const int32_t* entry, const int32_t* kinfo,
                     const int32_t* count, const int32_t* fmt, const int32_t* slot, int batch, int hk, int maxn,
                     int per, int tiles_max, const int32_t* bounds, int nsplit, const int32_t* items, int n_items,
                     int32_t* tasks, void* stream) {
  g_error.clear();
  if (!ka || !entry || !kinfo || !count || !fmt || !slot || !tasks) return fail("decode_tasks: null buffer");
  if (batch < 1 || hk < 1 || maxn < 1 || tiles_max < 1) return fail("decode_tasks: empty shape");
  if (!bounds && (per < 1 || per > tri::MAX_PER)) return fail("decode_tasks: per (tiles per split) must be in [1, 64]");
  if (bounds && (nsplit < 1 || nsplit > 65535)) return fail("decode_tasks: nsplit must be in [1, 65535]");
  if (!aligned(tasks, 16) || !aligned(ka, 16) || (ka4 && !aligned(ka4, 16)))
    return fail("decode_tasks: the table and the K scales must be 16-byte aligned");
  const int splits = bounds ? nsplit : std::max(1, (maxn + per - 1) / per);
  const int64_t all = (int64_t)splits * hk * batch;
  if (all >= ((int64_t)1 << 31) / tri::TASK_WORDS) return fail("decode_tasks: too many splits x heads x sequences");
  if (items && (n_items < 1 || n_items > all)) return fail("decode_tasks: n_items must be in [1, splits x hk x batch]");
  const int64_t listed = items ? n_items : all;
  tri::DecodeArgs d = {};
  d.ka = ka;
  d.ka4 = ka4;
  d.entry = entry;
  d.kinfo = kinfo;
  d.count = count;
  d.fmt = fmt;
  d.slot = slot;
  d.hk = hk;
  d.maxn = maxn;
  d.per = per;
  d.tiles_max = tiles_max;
  d.bounds = bounds;
  d.splits = splits;
  d.total = all;
  tri::decode_tasks_kernel<<<dim3((unsigned)listed), 64, 0, static_cast<hipStream_t>(stream)>>>(d, items, tasks);
  return check_launch("decode_tasks");
}

int tri_cache_store(const int32_t* bands, const int32_t* exact, int batch, int hq, int hk, int t, int nx,
                    int xstride, const void* kp, const void* k4p, const float* ka, const float* ka4, const float* kstat,
                    const float* vstat, const void* v8p, const void* v4p, const void* kx, const void* vx, int row0,
                    int rows, int maxn, int tiles_max, int32_t* entry, int32_t* kinfo, int32_t* slot, int32_t* count,
                    int32_t* fmt, int32_t* prompt, int32_t* xslot, float* ka_c, float* ka4_c, float* kstat_c,
                    float* vstat_c, void* k8c, int64_t o8, int64_t cap8, void* k4c, int64_t o4, int64_t cap4,
                    void* v8c, int64_t ov8, int64_t capv8, void* v4c, int64_t ov4, int64_t capv4, void* kxc,
                    void* vxc, int64_t ox, int64_t capx, void* stream) {
  g_error.clear();
  const int tiles = (t + tri::BN - 1) / tri::BN;
  if (!bands || !kp || !ka || !kstat || !vstat || !v8p || !entry || !kinfo || !slot || !count || !fmt || !prompt ||
      !ka_c || !kstat_c || !vstat_c || !k8c || !v8c)
    return fail("cache_store: null buffer");
  if (batch < 1 || hq < 1 || hk < 1 || t < 1) return fail("cache_store: empty shape");
  if (hq % hk != 0 || hq / hk > tri::MAX_GROUP || hq > tri::STORE_MAX_HQ)
    return fail("cache_store: q heads must be a multiple of the kv heads, groups of at most 8, at most 256 q heads");
  if (tiles > tri::MAX_TILES) return fail("cache_store: at most 131072 tokens");
  if (row0 < 0 || (int64_t)row0 + batch > rows) return fail("cache_store: rows %d..%d beyond the %d allocated", row0,
                                                             row0 + batch - 1, rows);
  if (maxn < 1 || tiles_max < tiles) return fail("cache_store: maxn >= 1 and tiles_max >= the prompt's tiles");
  if (exact && (nx < 1 || nx > hk || !kx || !vx || !kxc || !vxc || !xslot))
    return fail("cache_store: exact heads need nx in [1, hk], KX/VX sources, destinations and xslot");
  if (exact && xstride < tiles) return fail("cache_store: xstride (records per exact head) below the prompt's tiles");
  if (o8 < 0 || o4 < 0 || ov8 < 0 || ov4 < 0 || ox < 0) return fail("cache_store: negative record offset");
  if ((k4c == nullptr) != (cap4 == 0) || (v4c == nullptr) != (capv4 == 0))
    return fail("cache_store: INT4 K / V destinations and capacities (both or neither)");
  // record slots: K slots in the 23-bit kinfo field, V and exact-record slots in int32
  if (cap8 > ((int64_t)1 << 23) || cap4 > ((int64_t)1 << 23) || capv8 >= ((int64_t)1 << 31) ||
      capv4 >= ((int64_t)1 << 31) || capx >= ((int64_t)1 << 31))
    return fail("cache_store: K record arrays hold at most 2^23 records, V and KX/VX arrays fewer than 2^31");
  for (const void* p : {kp, k4p, v8p, v4p, kx, vx, (const void*)k8c, (const void*)k4c, (const void*)v8c,
                        (const void*)v4c, (const void*)kxc, (const void*)vxc})
    if (p && !aligned(p, 16)) return fail("cache_store: record arrays must be 16-byte aligned");
  tri::CacheStoreArgs a;
  a.bands = bands;
  a.exact = exact;
  a.hq = hq;
  a.hk = hk;
  a.t = t;
  a.tiles = tiles;
  a.nx = exact ? nx : 0;
  a.xstride = exact ? xstride : 0;
  a.batch = batch;
  a.kp = static_cast<const uint8_t*>(kp);
  a.k4p = static_cast<const uint8_t*>(k4p);
  a.v8p = static_cast<const uint8_t*>(v8p);
  a.v4p = static_cast<const uint8_t*>(v4p);
  a.kx = static_cast<const uint8_t*>(kx);
  a.vx = static_cast<const uint8_t*>(vx);
  a.ka = ka;
  a.ka4 = ka4;
  a.kstat = kstat;
  a.vstat = vstat;
  a.row0 = row0;
  a.rows = rows;
  a.maxn = maxn;
  a.tiles_max = tiles_max;
  a.entry = entry;
  a.kinfo = kinfo;
  a.slot = slot;
  a.count = count;
  a.fmt = fmt;
  a.prompt = prompt;
  a.xslot = xslot;
  a.ka_c = ka_c;
  a.ka4_c = ka4_c;
  a.kstat_c = kstat_c;
  a.vstat_c = vstat_c;
  a.k8c = static_cast<uint8_t*>(k8c);
  a.k4c = static_cast<uint8_t*>(k4c);
  a.v8c = static_cast<uint8_t*>(v8c);
  a.v4c = static_cast<uint8_t*>(v4c);
  a.kxc = static_cast<uint8_t*>(kxc);
  a.vxc = static_cast<uint8_t*>(vxc);
  a.o8 = o8;
  a.o4 = o4;
  a.ov8 = ov8;
  a.ov4 = ov4;
  a.ox = ox;
  a.cap8 = cap8;
  a.cap4 = cap4;
  a.capv8 = capv8;
  a.capv4 = capv4;
  a.capx = exact ? capx : 0;
  const dim3 grid((tiles + tri::STORE_CHUNK - 1) / tri::STORE_CHUNK, hk, batch);
  tri::cache_store_kernel<<<grid, tri::STORE_THREADS, 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("cache_store");
}

int tri_tail_spill(const int64_t* step, int64_t* tail_base, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh,
                   int64_t t_st, int max_tail, int rows, int hk, int maxn, int tiles_max, const int32_t* grow, int cap,
                   const int32_t* prompt, const int32_t* xslot, int32_t* entry, int32_t* kinfo, int32_t* slot,
                   int32_t* count, const int32_t* count0, int32_t* fmt, float* ka, float* ka4, const float* kstat, const float* vstat,
                   void* k8c, int64_t n_k8, void* k4c, int64_t n_k4, void* v8c, int64_t n_v8, void* kxc, void* vxc,
                   int64_t n_kx, int32_t* tasks, int n_tasks, void* stream) {
  g_error.clear();
  if (!step || !tail_base || !ktail || !vtail || !grow || !prompt || !entry || !kinfo || !slot || !count || !count0 ||
      !fmt ||
      !ka || !kstat || !vstat || !k8c || !v8c)
    return fail("tail_spill: null buffer");
  if (rows < 1 || hk < 1 || maxn < 1 || tiles_max < 1 || cap < 0) return fail("tail_spill: empty shape");
  if (max_tail < tri::BN || max_tail > tri::MAX_TAIL)
    return fail("tail_spill: tail growth moves 64 tokens at a time: max_tail must be in [64, 1024]");
  if (!aligned(ktail, 16) || !aligned(vtail, 16) || (t_sb % 8) || (t_sh % 8) || (t_st % 8))
    return fail("tail_spill: tail buffers must be 16-byte aligned rows");
  if (!aligned(grow, 16) || !aligned(ka, 16) || (ka4 && !aligned(ka4, 16)) || (tasks && !aligned(tasks, 16)))
    return fail("tail_spill: grow, the K scales and the task table must be 16-byte aligned");
  if ((k4c == nullptr) != (ka4 == nullptr)) return fail("tail_spill: INT4 K records and scales (both or neither)");
  if (xslot && (!kxc || !vxc)) return fail("tail_spill: exact heads need KX/VX record arrays");
  if (tasks && n_tasks < 1) return fail("tail_spill: a task table needs n_tasks >= 1");
  if (n_k8 < 1 || n_v8 < 1 || n_k8 > ((int64_t)1 << 23) || n_k4 > ((int64_t)1 << 23) || n_v8 >= ((int64_t)1 << 31) ||
      n_kx >= ((int64_t)1 << 31))
    return fail("tail_spill: record arrays must be non-empty, K arrays of at most 2^23 records");
  for (const void* p : {(const void*)k8c, (const void*)k4c, (const void*)v8c, (const void*)kxc, (const void*)vxc})
    if (p && !aligned(p, 16)) return fail("tail_spill: record arrays must be 16-byte aligned");
  tri::SpillArgs a;
  a.step = step;
  a.tail_base = tail_base;
  a.ktail = static_cast<uint16_t*>(ktail);
  a.vtail = static_cast<uint16_t*>(vtail);
  a.tsb = t_sb;
  a.tsh = t_sh;
  a.tst = t_st;
  a.max_tail = max_tail;
  a.rows = rows;
  a.hk = hk;
  a.maxn = maxn;
  a.tiles_max = tiles_max;
  a.cap = cap;
  a.grow = grow;
  a.prompt = prompt;
  a.xslot = xslot;
  a.entry = entry;
  a.kinfo = kinfo;
  a.slot = slot;
  a.count = count;
  a.count0 = count0;
  a.fmt = fmt;
  a.ka = ka;
  a.ka4 = ka4;
  a.kstat = kstat;
  a.vstat = vstat;
  a.k8c = static_cast<uint8_t*>(k8c);
  a.k4c = static_cast<uint8_t*>(k4c);
  a.v8c = static_cast<uint8_t*>(v8c);
  a.kxc = static_cast<uint8_t*>(kxc);
  a.vxc = static_cast<uint8_t*>(vxc);
  a.n_k8 = n_k8;
  a.n_k4 = k4c ? n_k4 : 0;
  a.n_v8 = n_v8;
  a.n_kx = xslot ? n_kx : 0;
  a.tasks = tasks;
  a.n_tasks = tasks ? n_tasks : 0;
  tri::tail_spill_kernel<<<dim3(hk, rows), tri::SPILL_THREADS, 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("tail_spill");
}

int tri_decode_occupancy(int* blocks) {
  g_error.clear();
  if (!blocks) return fail("decode_occupancy: null output");
  int n = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, tri::decode_kernel<4, false, false>, 64, 0);
  if (e != hipSuccess) return fail("decode_occupancy: %s", hipGetErrorString(e));
  *blocks = n;
  return 0;
}

int tri_device_cus(int* cus) {
  g_error.clear();
  if (!cus) return fail("device_cus: null output");
  return device_cus(cus);
}

int tri_prefill_pairs(int mode) {
  g_error.clear();
  if (mode < 0 || mode > 2) return fail("prefill_pairs: mode must be 0, 1 or 2 (got %d)", mode);
  g_prefill_pairs.store(mode);
  return 0;
}

int tri_stream_read(const void* base, int64_t records, int waves, int waves_per_group, int depth, int32_t* sink,
                    void* stream) {
  g_error.clear();
  if (!base || !sink) return fail("stream_read: null pointer");
  if (records <= 0 || waves <= 0) return fail("stream_read: records and waves must be positive");
  if (waves_per_group != 1 && waves_per_group != 2 && waves_per_group != 4)
    return fail("stream_read: waves_per_group must be 1, 2 or 4 (got %d)", waves_per_group);
  if (depth < 1 || depth > 3) return fail("stream_read: depth must be 1, 2 or 3 (got %d)", depth);
  const int64_t per = (records + waves - 1) / waves;
  if (per > INT32_MAX) return fail("stream_read: too many records per wave");
  const dim3 grid((waves + waves_per_group - 1) / waves_per_group), block(64 * waves_per_group);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* p = static_cast<const uint8_t*>(base);
  if (depth == 1) tri::stream_read_kernel<1><<<grid, block, 0, s>>>(p, records, (int)per, sink);
  else if (depth == 2) tri::stream_read_kernel<2><<<grid, block, 0, s>>>(p, records, (int)per, sink);
  else tri::stream_read_kernel<3><<<grid, block, 0, s>>>(p, records, (int)per, sink);
  return check_launch("stream_read");
}

int tri_issue_probe(int mode, int waves_per_simd, int iters, int64_t* out, void* stream) {
  g_error.clear();
  if (!out) return fail("issue_probe: null output");
  if (mode < 0 || mode >= tri::ISSUE_MODES) return fail("issue_probe: mode must be in [0, %d)", tri::ISSUE_MODES);
  if (waves_per_simd < 1 || waves_per_simd > 4) return fail("issue_probe: waves per SIMD must be 1..4");
  if (mode == 6 && waves_per_simd < 2) return fail("issue_probe: mode 6 needs at least two waves per SIMD");
  if (iters < 1 || iters > (1 << 20)) return fail("issue_probe: iterations must be in [1, 2^20]");
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return fail("issue_probe: no device");
  using K = void (*)(int, int64_t*, float, float, int);
  static const K kernels[tri::ISSUE_MODES] = {tri::issue_probe_kernel<0>, tri::issue_probe_kernel<1>,
                                             tri::issue_probe_kernel<2>, tri::issue_probe_kernel<3>,
                                             tri::issue_probe_kernel<4>, tri::issue_probe_kernel<5>,
                                             tri::issue_probe_kernel<6>, tri::issue_probe_kernel<7>,
                                             tri::issue_probe_kernel<8>, tri::issue_probe_kernel<9>,
                                             tri::issue_probe_kernel<10>, tri::issue_probe_kernel<11>,
                                             tri::issue_probe_kernel<12>, tri::issue_probe_kernel<13>,
                                             tri::issue_probe_kernel<14>};
  // 100 KiB of LDS per workgroup: at most one workgroup per CU
  constexpr int LDS = 100 * 1024;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernels[mode]), hipFuncAttributeMaxDynamicSharedMemorySize,
                          LDS) != hipSuccess)
    return fail("issue_probe: hipFuncSetAttribute");
  hipLaunchKernelGGL(kernels[mode], dim3(cus), dim3(256 * waves_per_simd), LDS, static_cast<hipStream_t>(stream), iters,
                     out, 1.0001f, 0.5f, 3);
  return check_launch("issue_probe");
}

}  // extern "C"
