/*
 * C ABI of the MI355X (gfx950) TriAttention kernels.
 *
 * Every entry point replaces one op of the reference's pybind module
 * (triattention/kernels/cuda/common_host.cuh:96-102), with tensors passed as
 * device pointers plus explicit sizes and element strides, and with a leading
 * batch dimension (batch = 1 is the reference's semantics exactly).  All
 * buffers are allocated by the caller; no entry point allocates.  Work is
 * enqueued asynchronously on `stream` (a hipStream_t; NULL = default stream).
 *
 * Return value: 0 on success, non-zero on a validation or launch error, with
 * a message available from tri_last_error() (thread-local).
 *
 * Record formats per (sequence, KV head, 64-key tile) keep the reference's
 * sizes: K8 8192 B, K4 4096 B, V16 16384 B, V8 8192 B, V4 4096 B, plus four
 * fp32 group scales per K tile (decode.py:7-8, prefill_sm80.cu:17-22).
 */
#ifndef TRIATTENTION_AMD_H
#define TRIATTENTION_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread ("" if none). */
const char* tri_last_error(void);

/* Replaces prepare_qk (common_host.cuh:1-25).
 * q: bf16 [batch][hq][t][128] with element strides (q_sb, q_sh, q_st), feature stride 1.
 * k: bf16 [batch][hk][t][128] likewise.
 * Outputs: q8 int8 [batch][hq][t][128], qa f32 [batch][hq][t], kp K8 records
 * [batch][hk][tiles], ka f32 [batch][hk][tiles][4], partial f32 scratch
 * [batch][hk][64][3][128], kstat f32 [batch][hk][3][128] (mean, scale, 1/scale).
 * q4/qa4/k4p/ka4 are all NULL or all set: q4 u8 [batch][hq][t][64] (low nibble =
 * even feature), qa4 f32 [batch][hq][t], k4p K4 records, ka4 f32 [batch][hk][tiles][4].
 * Extension: k4x (NULL, or with the INT4 buffers) receives the K4 records once more, each code
 * expanded to a byte of 16 * code in the K8 record layout (8 KiB per tile), for tri_attention's k4x. */
int tri_prepare_qk(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb,
                   int64_t k_sh, int64_t k_st, int batch, int hq, int hk, int t, void* q8, float* qa, void* kp,
                   float* ka, float* partial, float* kstat, void* q4, float* qa4, void* k4p, float* ka4,
                   void* k4x, void* stream);

/* Replaces pack_v (common_host.cuh:27-45).
 * v: bf16 [batch][hk][t][128]; vstat f32 [batch][hk][3][128].  Statistics are
 * the identity (0, 1, 1) when both v8p and v4p are NULL (common_host.cuh:39).
 * v16p/v8p/v4p: V16/V8/V4 records [batch][hk][tiles] or NULL.
 * v8sum (extension; NULL, or with v8p, 16-byte aligned): int32 [batch][hk][tiles][128], -127 times
 * each channel's sum of the tile's 64 V8 codes, for tri_attention's v8sum. */
int tri_pack_v(const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int batch, int hk, int t, float* partial,
               float* vstat, void* v16p, void* v8p, void* v4p, int32_t* v8sum, void* stream);

/* Replaces attention (prefill_sm80.cu:510-543), band-table form only (the
 * reference's task-table form has no caller, prefill.py:103).
 * order int32 [n_order = hq*tiles]: workgroup -> qhead*tiles + qtile.
 * bands int32 [hq][2] = (w8, w4) per q-head, shared by every sequence.
 * out: [batch][hq][t][128] with element strides (o_sb, o_sh, o_st), feature
 * stride 1; out_dtype 0 = fp32, 1 = bf16, 2 = fp16.  scale is the softmax
 * scale; sm_log2 = f32(scale * log2(e)) as in prefill_sm80.cu:538.
 * v16p/v8p/k8p/k4p records and ka8/ka4 scales must be 16-byte aligned; v8p
 * must be set whenever a band has INT8 or INT4 key tiles (both use INT8 V).
 * exact: NULL, or int32 [hq] on the device: 0 for a quantized q-head, else
 * 1 + the record slot (< nx) of its KV head.  Such a q-head ignores its band
 * and computes exact causal attention of the raw bf16 qr [batch][hq][t][128]
 * (strides q_sb, q_sh, q_st; rows 16-byte aligned) against the KX/VX records
 * [batch][nx][tiles] that tri_pack_exact wrote, with fp32 softmax and
 * accumulation (extension for maps that keep some heads unquantized).
 * v8sum (extension): NULL, or what tri_pack_v wrote for these V8 records; the
 * P V product of each INT8/INT4 tile then starts from it instead of computing
 * it with two MFMAs per 32 channels (the same integers either way).
 * k4x (extension): NULL, or what tri_prepare_qk wrote as k4x for these K4
 * records; INT4 key tiles then read those bytes instead of expanding the packed
 * nibbles in every tile (the same integers either way). */
int tri_attention(const int32_t* order, int n_order, const int32_t* bands, int batch, int hq, int hk, int t,
                  const void* v16p, const void* v8p, const float* vstat, const void* q8, const void* k8p,
                  const float* qa8, const float* ka8, const void* q4, const void* k4p, const float* qa4,
                  const float* ka4, void* out, int out_dtype, int64_t o_sb, int64_t o_sh, int64_t o_st,
                  double scale, const int32_t* exact, const void* qr, int64_t q_sb, int64_t q_sh, int64_t q_st,
                  const void* kx, const void* vx, int nx, const int32_t* v8sum, const void* k4x, void* stream);

/* No counterpart in the reference: the bf16 records of the exact heads that
 * tri_attention reads (extension).  k/v bf16 [batch][hk][t][128] with element
 * strides (rows 16-byte aligned); exact int32 [hq] as for tri_attention; the
 * KV head of q-head h*(hq/hk) with exact value s > 0 is written to slot s-1 of
 * kx/vx, 16 KiB per (sequence, slot, tile), keys at or past t zero.  Other KV
 * heads are not read. */
int tri_pack_exact(const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb,
                   int64_t v_sh, int64_t v_st, int batch, int hq, int hk, int t, const int32_t* exact, int nx,
                   void* kx, void* vx, void* stream);

/* Replaces decode (common_host.cuh:47-87), batched and ragged.  The merge takes its form on the
 * device: one wave per (sequence, q-head), in the reference's order (common_device.cuh:373-469), while
 * the tail (from *step and *tail_base) holds at most 16 tokens and batch * hq is at least twice the
 * device's CU count, four waves otherwise (within fp32 rounding of it); a captured graph replayed at
 * later steps therefore takes the form an eager call would take at every step.
 * q bf16 [batch][hq][1][128] (strides q_sb, q_sh); k8c/k4c/v8c/v4c compacted
 * records; ka/ka4 f32 [batch][hk][tiles_max][4]; entry/kinfo/slot int32
 * [batch][hk][maxn] (kinfo = rowmask | is4 << 8 | kslot << 9); count int32
 * [batch][hk]; fmt int32 [batch][tiles_max] (1 = INT8 V, 2 = INT4 V); prompt
 * int32 [batch] lengths; vstat/kstat f32 [batch][hk][3][128]; ktail/vtail bf16
 * [batch][hk][max_tail][128] (strides t_sb, t_sh, t_st); kcur/vcur bf16
 * [batch][hk][1][128] (strides c_sb, c_sh); tail and new-token rows 16-byte
 * aligned (strides multiples of 8 elements); step int64 [1] on the device;
 * out [batch][hq][1][128] (strides o_sb, o_sh), out_dtype 0 = fp32, 1 = bf16;
 * pm/pl f32 [batch][hq][splits], po f32 [batch][hq][splits][128] with
 * splits = max(1, ceil(maxn / per)) with 1 <= per <= 64; n_k8/n_k4/n_v8/n_v4 are the record
 * counts of the compacted arrays (K arrays at most 2^23 records, the kinfo slot field; every record is
 * addressed through its own 64-bit base, so no 32-bit byte-offset limit applies).
 * Exact (bf16) KV heads (extension): xslot NULL, or int32 [batch][hk] with -1
 * for a quantized head and otherwise the index of the head's first KX/VX
 * record in kxc/vxc (tri_pack_exact layout, n_kx records of 16 KiB each); such
 * a head keeps every prompt tile (count = tiles, entry[e] = e) and attends
 * exactly over its bf16 prompt and tail.
 * Entry words (extension): bits 0-28 hold the tile index; when bit 30 is set,
 * bit 29 holds the tile's V format (1 = INT8 V) and must agree with fmt, and the
 * kernel then starts streaming a split's first V record one memory round trip
 * earlier (reference-style entries, bits 29-30 clear, read fmt).
 * Split partition (extension): bounds NULL splits every head's kept tiles into
 * runs of `per` (the reference's split); otherwise bounds is int32
 * [batch][hk][nsplit + 1] and split s of a head covers entries
 * [bounds[s], bounds[s + 1]) (nondecreasing, bounds[0] = 0, bounds[nsplit] =
 * count, at most 64 entries per split), pm/pl/po then hold splits = nsplit.
 * Task table (extension): tasks NULL, or a table of n_tasks splits that tri_decode_tasks wrote for the
 * same ka / ka4 / entry / kinfo / count / fmt / slot / per / bounds.  The split kernel then runs only the
 * listed splits and reads each one's entries, record offsets and K scales from the table (one memory
 * round trip) instead of gathering them; the partials of splits the table leaves out are not written,
 * so the caller holds them at the empty partial (pm = -FLT_MAX, pl = 0, po = 0).  Ignored for a cache
 * with exact heads (xslot set).
 * Tail growth (extension): tail_base NULL keeps the reference's tail (it holds step tokens before the
 * new one, and past max_tail - 1 the new token overwrites the last slot, common_device.cuh:384);
 * otherwise int64 on the device, the tokens tri_tail_spill has moved from the tail into the cache since
 * the store, and the tail holds step - *tail_base tokens.  Tiles past a sequence's prompt tiles
 * (ceil(prompt / 64)) hold 64 valid keys each. */
int tri_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c, const float* ka,
               const float* ka4, const int32_t* entry, const int32_t* kinfo, const int32_t* count,
               const int32_t* fmt, const int32_t* slot, const void* v8c, const void* v4c, const float* vstat,
               const float* kstat, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh, int64_t t_st,
               int max_tail, const void* kcur, const void* vcur, int64_t c_sb, int64_t c_sh, const int64_t* step,
               void* out, int out_dtype, int64_t o_sb, int64_t o_sh, float* pm, float* pl, float* po,
               const int32_t* prompt, int batch, int hq, int hk, int maxn, int per, int tiles_max,
               int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4, const int32_t* xslot, const void* kxc,
               const void* vxc, int64_t n_kx, const int32_t* bounds, int nsplit, const void* tasks, int n_tasks, const int64_t* tail_base, double scale,
               void* stream);

/* The two launches of tri_decode separately, same arguments: the split-KV
 * kernel (writes pm/pl/po) and the merge with the bf16 tail (writes out and
 * appends kcur/vcur to the tail).  No reference counterpart; they let a caller
 * time or schedule the two kernels individually. */
int tri_decode_partials(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c,
                        const float* ka, const float* ka4, const int32_t* entry, const int32_t* kinfo,
                        const int32_t* count, const int32_t* fmt, const int32_t* slot, const void* v8c,
                        const void* v4c, const float* vstat, const float* kstat, void* ktail, void* vtail,
                        int64_t t_sb, int64_t t_sh, int64_t t_st, int max_tail, const void* kcur, const void* vcur,
                        int64_t c_sb, int64_t c_sh, const int64_t* step, void* out, int out_dtype, int64_t o_sb,
                        int64_t o_sh, float* pm, float* pl, float* po, const int32_t* prompt, int batch, int hq,
                        int hk, int maxn, int per, int tiles_max, int64_t n_k8, int64_t n_k4, int64_t n_v8,
                        int64_t n_v4, const int32_t* xslot, const void* kxc, const void* vxc, int64_t n_kx,
                        const int32_t* bounds, int nsplit, const void* tasks, int n_tasks, const int64_t* tail_base, double scale, void* stream);
int tri_decode_merge(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c, const float* ka,
                     const float* ka4, const int32_t* entry, const int32_t* kinfo, const int32_t* count,
                     const int32_t* fmt, const int32_t* slot, const void* v8c, const void* v4c, const float* vstat,
                     const float* kstat, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh, int64_t t_st,
                     int max_tail, const void* kcur, const void* vcur, int64_t c_sb, int64_t c_sh,
                     const int64_t* step, void* out, int out_dtype, int64_t o_sb, int64_t o_sh, float* pm, float* pl,
                     float* po, const int32_t* prompt, int batch, int hq, int hk, int maxn, int per, int tiles_max,
                     int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4, const int32_t* xslot, const void* kxc,
                     const void* vxc, int64_t n_kx, const int32_t* bounds, int nsplit, const void* tasks, int n_tasks, const int64_t* tail_base, double scale,
                     void* stream);

/* tri_decode and tri_decode_merge with the merge run as one wave per (sequence, q-head) whatever the
 * tail and grid: no reference counterpart.  Every load of the first 64 tail tokens and 16 splits is
 * issued at once and no workgroup barrier is needed, so on a grid of at least two (sequence, q-head)
 * workgroups per CU it is the faster merge while the tail (the step minus the tokens moved into the
 * cache) holds at most 16 tokens; any tail length gives a correct result, longer ones more slowly.
 * Its arithmetic follows the reference's merge order (common_device.cuh:373-469) exactly: tail scores
 * as 32-lane butterfly sums, split sums in four interleaved groups, tail tokens one after another.
 * tri_decode's merge takes this form by itself (chosen on the device) under those two conditions, with
 * the same bits.  Same arguments as tri_decode. */
int tri_decode_short_tail(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c,
                          const float* ka, const float* ka4, const int32_t* entry, const int32_t* kinfo,
                          const int32_t* count, const int32_t* fmt, const int32_t* slot, const void* v8c,
                          const void* v4c, const float* vstat, const float* kstat, void* ktail, void* vtail,
                          int64_t t_sb, int64_t t_sh, int64_t t_st, int max_tail, const void* kcur, const void* vcur,
                          int64_t c_sb, int64_t c_sh, const int64_t* step, void* out, int out_dtype, int64_t o_sb,
                          int64_t o_sh, float* pm, float* pl, float* po, const int32_t* prompt, int batch, int hq,
                          int hk, int maxn, int per, int tiles_max, int64_t n_k8, int64_t n_k4, int64_t n_v8,
                          int64_t n_v4, const int32_t* xslot, const void* kxc, const void* vxc, int64_t n_kx,
                          const int32_t* bounds, int nsplit, const void* tasks, int n_tasks, const int64_t* tail_base,
                          double scale, void* stream);
int tri_decode_merge_short_tail(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c,
                          const float* ka, const float* ka4, const int32_t* entry, const int32_t* kinfo,
                          const int32_t* count, const int32_t* fmt, const int32_t* slot, const void* v8c,
                          const void* v4c, const float* vstat, const float* kstat, void* ktail, void* vtail,
                          int64_t t_sb, int64_t t_sh, int64_t t_st, int max_tail, const void* kcur, const void* vcur,
                          int64_t c_sb, int64_t c_sh, const int64_t* step, void* out, int out_dtype, int64_t o_sb,
                          int64_t o_sh, float* pm, float* pl, float* po, const int32_t* prompt, int batch, int hq,
                          int hk, int maxn, int per, int tiles_max, int64_t n_k8, int64_t n_k4, int64_t n_v8,
                          int64_t n_v4, const int32_t* xslot, const void* kxc, const void* vxc, int64_t n_kx,
                          const int32_t* bounds, int nsplit, const void* tasks, int n_tasks, const int64_t* tail_base,
                          double scale, void* stream);

/* Measurement (no reference counterpart): tri_decode_partials with the split-KV
 * kernel launched through hipExtLaunchKernel, which records the two hipEvent_t
 * handles (either may be null) as the kernel's own start and stop, so that a
 * caller can time the kernel without event commands of its own in the stream. */
int tri_decode_partials_timed(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c,
                              const float* ka, const float* ka4, const int32_t* entry, const int32_t* kinfo,
                              const int32_t* count, const int32_t* fmt, const int32_t* slot, const void* v8c,
                              const void* v4c, const float* vstat, const float* kstat, void* ktail, void* vtail,
                              int64_t t_sb, int64_t t_sh, int64_t t_st, int max_tail, const void* kcur,
                              const void* vcur, int64_t c_sb, int64_t c_sh, const int64_t* step, void* out,
                              int out_dtype, int64_t o_sb, int64_t o_sh, float* pm, float* pl, float* po,
                              const int32_t* prompt, int batch, int hq, int hk, int maxn, int per,
                              int tiles_max, int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4,
                              const int32_t* xslot, const void* kxc, const void* vxc, int64_t n_kx,
                              const int32_t* bounds, int nsplit, const void* tasks, int n_tasks, const int64_t* tail_base, double scale, void* stream, void* ev_start,
                              void* ev_stop);

/* No counterpart in the reference: the split kernel's task table for a decode cache's current layout.
 * Work items are (sequence, KV head, split) of the split tri_decode makes from per / bounds (splits =
 * nsplit with bounds, else max(1, ceil(maxn / per))), numbered ((sequence * hk) + head) * splits + split.
 * For the i-th of the n_items items listed in items (int32 on the device; NULL lists every item in
 * order), 512 int32 at tasks + i * 512: an int4 per lane L (K record slot, V record
 * slot, rowmask | INT4-K << 8 | INT8-V << 9 | tile << 10, and the work item in lane 0 / the split's
 * entry count in the other lanes) for the split's entry L, then a float4 per lane (the tile's K group
 * scales).  16-byte aligned.  Rebuild it whenever the cache or its split partition changes. */
int tri_decode_tasks(const float* ka, const float* ka4, const int32_t* entry, const int32_t* kinfo,
                     const int32_t* count, const int32_t* fmt, const int32_t* slot, int batch, int hk, int maxn,
                     int per, int tiles_max, const int32_t* bounds, int nsplit, const int32_t* items, int n_items,
                     int32_t* tasks, void* stream);

/* Replaces the host-side assembly of DecodeCache.store (kernels/decode.py:24-67): one launch appends
 * the decode-cache entries of a Prefill call's batch (batch sequences of t tokens each) as rows row0 ..
 * row0 + batch - 1 of a cache with `rows` rows, computing the kept-tile metadata on the device from
 * bands int32 [hq][2] and compacting the records.
 * Sources (the Prefill outputs): kp / k4p K8 / K4 records, v8p / v4p V8 / V4 records [batch][hk][tiles],
 * ka / ka4 f32 [batch][hk][tiles][4], kstat / vstat f32 [batch][hk][3][128]; k4p / ka4 / v4p may be NULL
 * when no tile needs them.  exact: NULL, or int32 [hk] on the device, -1 for a quantized KV head and
 * otherwise the head's slot (< nx) in kx / vx [batch][nx][tiles] (16 KiB bf16 records, tri_pack_exact);
 * in kxc / vxc each (sequence, exact head) takes xstride >= tiles records (room for tiles that
 * tri_tail_spill appends).
 * Destinations, as tri_decode reads them: entry / kinfo / slot [rows][hk][maxn] (entries past a head's
 * count zero), count [rows][hk], fmt [rows][tiles_max] (1 = INT8 V, 2 = INT4 V, 1 past the prompt),
 * prompt [rows], xslot [rows][hk] (may be NULL without exact heads), ka_c / ka4_c [rows][hk][tiles_max][4]
 * (1.0 past the prompt; ka4_c may be NULL), kstat_c / vstat_c [rows][hk][3][128], and the compacted
 * record arrays k8c / k4c / v8c / v4c / kxc / vxc whose first free records are o8 / o4 / ov8 / ov4 / ox
 * and which hold cap8 / cap4 / capv8 / capv4 / capx records (records past a capacity are not written;
 * k4c / v4c NULL with capacity 0 when absent).  Within a sequence, records are numbered in (KV head,
 * entry) order and each sequence takes as many as its metadata selects, after the previous sequence's. */
int tri_cache_store(const int32_t* bands, const int32_t* exact, int batch, int hq, int hk, int t, int nx,
                    int xstride, const void* kp, const void* k4p, const float* ka, const float* ka4, const float* kstat,
                    const float* vstat, const void* v8p, const void* v4p, const void* kx, const void* vx, int row0,
                    int rows, int maxn, int tiles_max, int32_t* entry, int32_t* kinfo, int32_t* slot, int32_t* count,
                    int32_t* fmt, int32_t* prompt, int32_t* xslot, float* ka_c, float* ka4_c, float* kstat_c,
                    float* vstat_c, void* k8c, int64_t o8, int64_t cap8, void* k4c, int64_t o4, int64_t cap4,
                    void* v8c, int64_t ov8, int64_t capv8, void* v4c, int64_t ov4, int64_t capv4, void* kxc,
                    void* vxc, int64_t ox, int64_t capx, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): tri_decode with the split
 * partials pm / pl / po held in a scratch array inside the library (24 MiB of fp32 per GPU, held until
 * the process ends) instead of caller buffers; every other argument as for tri_decode, and the
 * same kernels.  Calls whose batch x hq x splits partials do not fit (more than 48,395) are rejected
 * with an error.  No memory is allocated or freed.  Every call on one GPU shares that GPU's scratch
 * (each call writes every partial it reads).  Calls on one stream are ordered by the stream; a call
 * on another stream while the last call's work is still pending is refused with an error (the library
 * records an event after each call; it creates that event, with the scratch address, at its first call
 * on a device).  A call made under stream capture is not checked: replays of a graph that holds it
 * must not overlap calls on other streams. */
int tri_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh, const void* k8c, const void* k4c, const float* ka,
                       const float* ka4, const int32_t* entry, const int32_t* kinfo, const int32_t* count,
                       const int32_t* fmt, const int32_t* slot, const void* v8c, const void* v4c, const float* vstat,
                       const float* kstat, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh, int64_t t_st,
                       int max_tail, const void* kcur, const void* vcur, int64_t c_sb, int64_t c_sh,
                       const int64_t* step, void* out, int out_dtype, int64_t o_sb, int64_t o_sh,
                       const int32_t* prompt, int batch, int hq, int hk, int maxn, int per, int tiles_max,
                       int64_t n_k8, int64_t n_k4, int64_t n_v8, int64_t n_v4, const int32_t* xslot,
                       const void* kxc, const void* vxc, int64_t n_kx, const int32_t* bounds, int nsplit,
                       const void* tasks, int n_tasks, const int64_t* tail_base, double scale, void* stream);

/* No counterpart in the reference, which overwrites the tail's last slot once max_tail tokens are
 * generated (common_device.cuh:384): tail growth for one layer's decode cache, launched before each of
 * the layer's tri_decode calls.  When the tail holds max_tail tokens (*step - tail_base[0] >= max_tail,
 * max_tail >= 64), the oldest 64 tail tokens of every (sequence, KV head) become a new tile of the cache
 * and the tail moves up by 64 slots; tail_base[0] then grows by 64 (int64 [2] on the device, zero at the
 * store; tail_base[1] is the kernel's own counter and must stay zero between launches).  Otherwise
 * nothing is written.  The new tile is tile ceil(prompt / 64) + tail_base[0] / 64 of its sequence,
 * quantized with the prompt's statistics (INT8 or INT4 K with four group scales, INT8 V) and classified
 * as the newest tile of the cache; an exact head (xslot >= 0) stores KX / VX records at xslot + tile.
 * grow int32 [rows][hk][4] per (sequence, KV head): the new tile's kinfo bits (rowmask | INT4 K << 8,
 * or -1 when no q-head keeps it), the K and V record slots of its first spilled tile (spill n uses
 * slot + n), and the task-table row of its first growth split (-1: none; growth split i holds spilled
 * tiles 64 i .. 64 i + 63 as entries count0 + 64 i ...).  cap: spilled tiles per head that the arrays
 * have room for (when full, nothing moves and the tail clamps as the reference's does).  count0
 * [rows][hk]: each head's entry count at the store.  A spill happens for all (sequence, KV head) pairs
 * or for none: when any pair lacks room for the tile (tile index >= tiles_max, count0 + spills >= maxn,
 * a record slot past n_k8 / n_k4 / n_v8 / n_kx, or INT4 K without k4c / ka4), nothing is written and
 * the tail clamps as at cap.  The metadata arrays, K scales and records are the cache's, as tri_decode
 * reads them; tasks (may be NULL) is its task table. */
int tri_tail_spill(const int64_t* step, int64_t* tail_base, void* ktail, void* vtail, int64_t t_sb, int64_t t_sh,
                   int64_t t_st, int max_tail, int rows, int hk, int maxn, int tiles_max, const int32_t* grow, int cap,
                   const int32_t* prompt, const int32_t* xslot, int32_t* entry, int32_t* kinfo, int32_t* slot,
                   int32_t* count, const int32_t* count0, int32_t* fmt, float* ka, float* ka4, const float* kstat,
                   const float* vstat, void* k8c, int64_t n_k8, void* k4c, int64_t n_k4, void* v8c, int64_t n_v8,
                   void* kxc, void* vxc, int64_t n_kx, int32_t* tasks, int n_tasks, void* stream);

/* Replaces decode_occupancy (common_host.cuh:89-94): resident decode
 * workgroups per compute unit, written to *blocks. */
int tri_decode_occupancy(int* blocks);

/* Compute units of the current device (used to size decode splits). */
int tri_device_cus(int* cus);

/* Extension, no counterpart in the reference: the launch form of tri_attention for this process.
 * mode 0 (default): launches with at most two workgroups per compute unit take four-wave workgroups
 * whose two wave pairs split each query tile's key tiles (the F16 tiles and the start of the
 * quantized list, and the rest), merged before the output; larger launches take two-wave
 * workgroups.  mode 1: always two-wave workgroups; mode 2: always four.  Both forms follow the
 * reference's per-tile arithmetic; they differ only in the fp32 summation order across the two
 * parts (tests hold both to the same bar).  Returns 1 for another mode. */
int tri_prefill_pairs(int mode);

/* Measurement aid, no counterpart in the reference: reads `records` records of 8192 bytes from
 * `base` with no compute (wave i takes a contiguous run of ceil(records / waves) records, `depth`
 * of them in flight, 16-byte loads per lane), the device's streaming-read ceiling against which
 * the decode kernel's record stream is measured.  waves_per_group 1, 2 or 4; depth 1..3; sink: one
 * int32 of device memory (never written in practice). */
int tri_stream_read(const void* base, int64_t records, int waves, int waves_per_group, int depth, int32_t* sink,
                    void* stream);

/* Measurement aid, no reference counterpart: the issue cost of the instruction kinds the attention
 * tiles are made of.  One workgroup per CU of 256 * waves_per_simd threads (1..4 waves per SIMD) runs
 * `iters` iterations of `mode` (0: 32 v_fma_f32; 1: 8 v_exp_f32; 2: 24 v_fma_f32 + 8 v_exp_f32;
 * 3: 4 v_mfma_i32_32x32x32_i8; 4: 4 v_mfma_f32_32x32x16_bf16; 5: 4 i8 MFMA + 64 v_fma_f32 in one wave;
 * 6: the first wave of each SIMD 4 i8 MFMA, the others 32 v_fma_f32; 7-12: 4 i8 MFMA and 96 v_fma_f32
 * per wave, 7 spread, 8 MFMAs first, 9 as 8 then a barrier, 10 as 9 with the fma after the MFMA results,
 * 11 as 10 with the odd waves of a SIMD half an iteration behind, 12 as 7 then a barrier; 13: a
 * tile-shaped iteration, 16 i8 MFMA interleaved with 128 v_fma_f32 then 200 v_fma_f32 and 32 v_exp_f32
 * after the MFMA results, then a barrier; 14: as 13 with the odd waves of a SIMD in the other order) and
 * writes, per wave
 * w = workgroup * 4 * waves_per_simd + wave, its elapsed shader-clock cycles (s_memtime) to out[2w]
 * and 100 MHz ticks (s_memrealtime) to out[2w + 1].  out: int64 [2 * CUs * 4 * waves_per_simd]. */
int tri_issue_probe(int mode, int waves_per_simd, int iters, int64_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIATTENTION_AMD_H */
