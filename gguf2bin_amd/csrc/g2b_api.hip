// g2b_api.hip - the C ABI of include/g2b_attn.h and include/g2b_synth.h.
//
// Host-side control of the decode-attention path: shape validation, KV
// buffers in HBM with the reference layout, the RoPE table (built on the host
// by g2b_rope_table), QK-RMSNorm weights, staging of batch descriptors,
// split sizing and the launches per call (k_layer + k_combine, or append,
// generic decode and combine for shapes without a specialised kernel).  Nothing here computes
// attention on the CPU: if the device path cannot run, the call fails.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <mutex>
#include <vector>

#include "g2b_attn.h"
#include "g2b_internal.h"
#include "g2b_limits.h"
#include "g2b_matmul.h"
#include "g2b_synth.h"

using namespace g2b;

struct g2b_ctx {
  int32_t device = 0;
  g2b_shape shape{};
  ShapeDev sh{};
  float qscale = 0.f;
  hipStream_t own = nullptr, stream = nullptr;

  float *rope = nullptr;  // [rope_len][head_dim]
  int32_t rope_len = 0;

  // current batch
  int32_t n_seq = 0, max_pos = 0;
  int64_t total_pos = 0;
  SeqDev *d_seqs = nullptr, *h_seqs = nullptr;  // h_seqs: pinned staging
  SeqDev seq0{};  // the batch's only sequence (n_seq == 1): passed by value
  int32_t seqs_cap = 0;
  uint64_t batch_gen = 0;  // counts g2b_batch_begin calls

  // work-queue home units (G2B_HOME_ENTRIES each): the table of the last
  // (batch, layers per call, grid) it was made for
  int32_t *home_d = nullptr, *home_h = nullptr;
  hipEvent_t home_ev = nullptr;
  bool home_ev_live = false;
  uint64_t home_key[3] = {0, 0, 0};
  hipEvent_t seqs_ev = nullptr;
  bool seqs_ev_live = false;

  // scratch
  float *qrot = nullptr;
  size_t qrot_cap = 0;  // floats
  float *part = nullptr;
  size_t part_cap = 0;
  float *hstage = nullptr;  // device staging for the *_host entry point
  size_t hstage_cap = 0;

  // QK-RMSNorm weights (g2b_set_qk_norm)
  float *qkn_w = nullptr;       // device [n_layers][2][head_dim]
  int32_t *qkn_on = nullptr;    // device [n_layers]: bit 0 q, bit 1 k
  std::vector<int32_t> qkn_on_h;
  float qkn_eps = 0.f;

  int32_t n_cu = 1;            // compute units of the device
  int32_t occ_cache[2][3][2];  // workgroups per CU by (half-block lanes, stage mode, work queue)
  int32_t split_override = 0;  // g2b_ctx_tune
  int32_t tune_chunk = 0;
  int32_t tune_piece = 0;      // -1: static splits only; > 0: work-queue piece length

  // work-queue counters of k_layer: two sets of wq_cap units (DecodeParams.wq)
  int32_t *wq = nullptr;
  int32_t wq_cap = 0, wq_set = 0;
  int32_t wq_dirty[2] = {0, 0};  // units of each set a launch may have left non-zero
  bool wq_reset = false;         // a launch failed after using the counters
  int32_t tune_stage = 0;      // -1: k_layer loads straight from HBM; 1, 2: staging mode
  int32_t tune_kernel = 0;     // 0 automatic, 1 k_layer only, 2 k_tiles, 3 spanned k_short
  int32_t *span_ctr = nullptr; // k_short's span tickets (zero between launches)
  size_t span_ctr_cap = 0;
  int32_t occ_tiles[2] = {0, 0};  // k_tiles workgroups per CU (static, work queue)

  // the last decode call's schedule (g2b_ctx_last_schedule)
  int32_t sched[G2B_SCHED_FIELDS] = {};

  // decode-launch timing (g2b_ctx_profile)
  bool prof = false;
  std::vector<hipEvent_t> prof_ev;  // pairs: [2i] before, [2i+1] after launch i
  size_t prof_used = 0;             // events used in the current window

  float *fixed = nullptr;  // this device's copy of `scratch` (g2b_attn_forward_noalloc)

  // phase stamps (DecodeParams.stamps; set only by the G2B_STAMPS build):
  // stamp_launches regions of 2 * stamp_cap * kStampWords words, decode call
  // i using region i % stamp_launches since the last read
  uint64_t *stamps = nullptr;
  int32_t stamp_cap = 0, stamp_launches = 0, stamp_next = 0;

  std::string err;
};

// Scratch of the allocation-free entry point g2b_attn_forward_noalloc: the
// split partials (and the generic path's rotated q) of its calls, in
// file-scope device memory instead of buffers the context allocates.  Each
// GPU the library runs on holds its own copy until the process ends; calls on
// one GPU share it (each call overwrites what it uses and reads nothing it did
// not write), so calls that overlap on one GPU race.  Host code never names
// the array itself (that is a host-side stand-in): it uses the address
// hipGetSymbolAddress gives per device, taken once per device at context
// creation.
constexpr size_t kFixedScratchBytes = (size_t)2 << 20;
static __device__ __align__(256) float scratch[kFixedScratchBytes / sizeof(float)];
// Its first kFixedCtrInts words are k_short's span counters: zero at load
// (static storage) and left zero by every launch; nothing else uses them.
constexpr size_t kFixedCtrInts = 1024;

namespace {

int fail(g2b_ctx *c, int code, const char *fmt, ...) {
  if (c) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
  }
  return code;
}

#define G2B_HIP(c, call)                                                          \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) return fail((c), G2B_EDEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

size_t row_bytes_of(const g2b_shape *s) {
  const size_t nkv = (size_t)s->n_kv_heads * (size_t)s->head_dim;
  return s->kv_q8 ? (nkv + 31u) / 32u * 34u : nkv * 4u;
}

constexpr size_t kKvSlack = G2B_KV_SLACK;
static_assert(sizeof(SeqDev) == G2B_SEQ_DESC_BYTES, "descriptor size the budget assumes");
static_assert(kPartHead == (int)G2B_PART_HEAD, "partial layout the budget assumes");
static_assert(kWqStride * sizeof(int32_t) == G2B_WQ_LINE_BYTES, "counter line the budget assumes");

// The staged KV loads read 16-byte pieces from the cache bases.
bool misaligned(const void *p) { return ((uintptr_t)p & 15u) != 0; }

int set_device(g2b_ctx *c) {
  G2B_HIP(c, hipSetDevice(c->device));
  return G2B_OK;
}

// This device's address of `scratch`, looked up once per device (the device
// must be current).
std::mutex g_fixed_mu;
std::vector<float *> g_fixed_ptr;  // by device id
hipError_t fixed_scratch_of(int32_t device, float **out) {
  std::lock_guard<std::mutex> lock(g_fixed_mu);
  if ((size_t)device >= g_fixed_ptr.size()) g_fixed_ptr.resize((size_t)device + 1, nullptr);
  if (!g_fixed_ptr[(size_t)device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_fixed_ptr[(size_t)device] = (float *)p;
  }
  *out = g_fixed_ptr[(size_t)device];
  return hipSuccess;
}

// Grow a device buffer (contents are not kept); waits for queued work first.
// Grows by half again at least, but never past limit_floats (>= need_floats),
// the size g2b_hbm_bytes budgets for the buffer.
int grow(g2b_ctx *c, float **buf, size_t *cap, size_t need_floats, size_t limit_floats) {
  if (*cap >= need_floats) return G2B_OK;
  size_t n = std::max(need_floats, std::min(*cap + *cap / 2, limit_floats));
  if (*buf) {
    G2B_HIP(c, hipStreamSynchronize(c->stream));
    G2B_HIP(c, hipFree(*buf));
    *buf = nullptr;
    *cap = 0;
  }
  if (hipMalloc((void **)buf, n * sizeof(float)) != hipSuccess) {
    *buf = nullptr;
    (void)hipGetLastError();
    return fail(c, G2B_ENOMEM, "hipMalloc of %zu bytes failed", n * sizeof(float));
  }
  *cap = n;
  return G2B_OK;
}

NormDev norm_of(const g2b_ctx *c) {
  NormDev n{};
  bool any = false;
  for (int32_t f : c->qkn_on_h) any |= f != 0;
  n.w = any ? c->qkn_w : nullptr;
  n.on = c->qkn_on;
  n.eps = c->qkn_eps;
  return n;
}

int ensure_rope(g2b_ctx *c, int32_t len) {
  if (!c->sh.rope_on || len <= c->rope_len) return G2B_OK;
  const int32_t n = std::max(len, std::max(c->rope_len * 2, 256));
  const size_t floats = (size_t)n * (size_t)c->shape.head_dim;
  float *host = (float *)malloc(floats * sizeof(float));
  if (!host) return fail(c, G2B_ENOMEM, "host RoPE table of %zu bytes", floats * 4);
  int rc = g2b_rope_table(0, n, c->shape.head_dim, c->shape.rope_theta, host);
  if (rc) {
    free(host);
    return fail(c, rc, "g2b_rope_table failed");
  }
  float *dev = nullptr;
  if (hipMalloc((void **)&dev, floats * sizeof(float)) != hipSuccess) {
    free(host);
    (void)hipGetLastError();
    return fail(c, G2B_ENOMEM, "hipMalloc RoPE table");
  }
  hipError_t e = hipMemcpy(dev, host, floats * sizeof(float), hipMemcpyHostToDevice);
  free(host);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return fail(c, G2B_EDEVICE, "RoPE table upload: %s", hipGetErrorString(e));
  }
  if (c->rope) {
    G2B_HIP(c, hipStreamSynchronize(c->stream));
    G2B_HIP(c, hipFree(c->rope));
  }
  c->rope = dev;
  c->rope_len = n;
  return G2B_OK;
}

// Positions per split.  The decode workgroups of one call should form whole
// rounds of the device's resident slots (CUs x workgroups per CU): with equal
// work per workgroup they start and finish together, and the launch has no
// partly idle tail.  One round when the work allows it; otherwise as many
// rounds as the minimum split length forces.  At most 512 splits per
// sequence (each is one partial per head for the combine, which stages a
// weight per partial in LDS) and the generic kernel's LDS limit apply.
// Resident k_layer workgroups on the device for the variant of dp (cached).
int32_t slots_for(g2b_ctx *c, const DecodeParams &dp, bool wq) {
  int32_t &occ = c->occ_cache[dp.tune_chunk == 16 ? 1 : 0][dp.stage_mode][wq ? 1 : 0];
  if (occ <= 0) occ = decode_blocks_per_cu(c->sh, dp.tune_chunk, dp.stage_mode, dp.stage_rows, wq);
  return std::max(1, c->n_cu) * std::max(1, occ);
}

// Resident k_tiles workgroups on the device (cached).
int32_t tiles_slots(g2b_ctx *c, bool wq) {
  int32_t &occ = c->occ_tiles[wq ? 1 : 0];
  if (occ <= 0) occ = tiles_blocks_per_cu(c->sh, wq);
  return std::max(1, c->n_cu) * std::max(1, occ);
}

// Positions per split of a static schedule.  min_len is the shortest split
// worth a workgroup (its waves get a few wave-steps or chunks each; shorter
// splits cost more in setup and partials than they gain).
//
// One sequence (every unit the same length): the launch's workgroups,
// n_layers * ceil((max_pos+1)/len), fill the fewest whole rounds of `slots`
// that the layers allow (one round for up to `slots` layers), with the
// shortest splits that fit.  Measured on the single-sequence calls: a launch
// a few workgroups past a round runs ~35% longer (c1, all layers: 90.8 us at
// 252 workgroups of 256 slots, 123 us at 308) and many rounds of short
// splits lose to one round of long ones (100 us at 924); the rule gives c1
// 252 workgroups (92.7 us, was 109) and c2 504 of 512 (97.5 us, was 131).
// Batches: the average work per slot, total_pos * n_layers / slots (ragged
// lengths make whole-round counting moot; measured on the 64-sequence SmolLM2
// F32 batch (c3), the round rule lost 20% layer-serial and 50% in one call).
int32_t choose_split(const g2b_ctx *c, int64_t slots, int32_t n_seq, int64_t total_pos,
                     int32_t max_pos, int32_t n_layers, bool fast, int32_t min_len) {
  const int64_t hi = (int64_t)max_pos + 1;
  const int64_t min_for_cap = (hi + 511) / 512;
  int64_t sl;
  if (c->split_override > 0) {
    sl = c->split_override;
  } else if (n_seq == 1) {
    const int64_t lo = std::min<int64_t>(std::max<int64_t>(min_len, min_for_cap), hi);
    const int64_t target = ((int64_t)n_layers + slots - 1) / slots * slots;
    // the per-layer split count that fits, then the shortest length giving it
    const int64_t per_layer = std::max<int64_t>(1, target / n_layers);
    sl = std::max<int64_t>(lo, (hi + per_layer - 1) / per_layer);
  } else {
    sl = std::max<int64_t>((total_pos * (int64_t)n_layers + slots - 1) / slots, min_len);
  }
  sl = std::max(sl, min_for_cap);
  if (!fast) sl = std::min<int64_t>(sl, kGenericMaxSplit);
  sl = std::min<int64_t>(sl, hi);
  return (int32_t)std::max<int64_t>(sl, 1);
}

// Zeroes device memory before anything on the context's stream can read it:
// the stream is non-blocking, so a hipMemset on the null stream would not be
// ordered before its launches.
int zero_device(g2b_ctx *c, void *p, size_t bytes) {
  G2B_HIP(c, hipMemsetAsync(p, 0, bytes, c->stream));
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  return G2B_OK;
}

// At least n of k_short's span tickets, zero between launches (the last span
// of each (sequence, layer, KV head) resets its own).
int span_counters(g2b_ctx *c, size_t n) {
  if (n <= c->span_ctr_cap) return G2B_OK;
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  if (c->span_ctr) G2B_HIP(c, hipFree(c->span_ctr));
  c->span_ctr = nullptr;
  c->span_ctr_cap = 0;
  const size_t cap = std::max<size_t>(n, G2B_SPAN_CTR_MIN);
  if (hipMalloc((void **)&c->span_ctr, cap * sizeof(int32_t)) != hipSuccess) {
    c->span_ctr = nullptr;
    (void)hipGetLastError();
    return fail(c, G2B_ENOMEM, "span counters");
  }
  c->span_ctr_cap = cap;
  if (int rc = zero_device(c, c->span_ctr, cap * sizeof(int32_t))) return rc;
  return G2B_OK;
}

void set_sched(g2b_ctx *c, int32_t kernel, int32_t split_len, int32_t piece_len,
               int32_t max_splits, int64_t grid, bool direct, int32_t staging = 0,
               int32_t chunk = 0, bool weights = false) {
  c->sched[0] = kernel;
  c->sched[1] = split_len;
  c->sched[2] = piece_len;
  c->sched[3] = max_splits;
  c->sched[4] = (int32_t)std::min<int64_t>(grid, INT32_MAX);
  c->sched[5] = direct ? 1 : 0;
  c->sched[6] = staging;
  c->sched[7] = chunk;
  c->sched[8] = weights ? 1 : 0;
}

// With g2b_ctx_profile on: records the first of two timing events around
// the next decode launch and hands back the second (*ev1), else *ev1 = null.
int prof_begin(g2b_ctx *c, hipEvent_t *ev1) {
  *ev1 = nullptr;
  if (!c->prof) return G2B_OK;
  if (c->prof_used + 2 > c->prof_ev.size()) {
    for (int i = 0; i < 2; i++) {
      hipEvent_t e;
      G2B_HIP(c, hipEventCreate(&e));
      c->prof_ev.push_back(e);
    }
  }
  const hipEvent_t ev0 = c->prof_ev[c->prof_used];
  *ev1 = c->prof_ev[c->prof_used + 1];
  c->prof_used += 2;
  G2B_HIP(c, hipEventRecord(ev0, c->stream));
  return G2B_OK;
}

// The work queue's first unit of each of `grid` workgroups, for a ragged
// batch (the host copy of its descriptors): every unit gets one workgroup,
// the rest go to the units in proportion to the positions they stream, so
// that the units run dry together instead of the short ones' workgroups
// moving to other units (a visit costs a setup) or leaving early.  Measured
// on c5 (32 sequences of 16k-32k positions, 512 workgroups): with 16
// workgroups per unit the workgroups finished between 269 and 348 us of a
// 352 us launch.  Made once per (batch, layers per call, grid) and uploaded
// on the stream; null when every unit has the same length or the grid has
// no more workgroups than units.
int wq_home_table(g2b_ctx *c, int32_t n_seq, int32_t n_layers, int64_t grid,
                  const int32_t **out) {
  *out = nullptr;
  const int64_t n_units = (int64_t)n_seq * n_layers;
  if (n_seq < 2 || grid <= n_units || grid > (int64_t)G2B_HOME_ENTRIES) return G2B_OK;
  bool same = true;
  for (int32_t i = 1; i < n_seq && same; i++) same = c->h_seqs[i].pos == c->h_seqs[0].pos;
  if (same) return G2B_OK;
  if (c->home_d && c->home_key[0] == c->batch_gen && c->home_key[1] == (uint64_t)n_layers &&
      c->home_key[2] == (uint64_t)grid) {
    *out = c->home_d;
    return G2B_OK;
  }
  if (!c->home_d) {
    if (hipMalloc((void **)&c->home_d, G2B_HOME_ENTRIES * sizeof(int32_t)) != hipSuccess ||
        hipHostMalloc((void **)&c->home_h, G2B_HOME_ENTRIES * sizeof(int32_t),
                      hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&c->home_ev, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      if (c->home_d) (void)hipFree(c->home_d);
      if (c->home_h) (void)hipHostFree(c->home_h);
      c->home_d = nullptr;
      c->home_h = nullptr;
      c->home_ev = nullptr;
      return fail(c, G2B_ENOMEM, "work-queue home table");
    }
  }
  // the previous upload must have read the staging buffer
  if (c->home_ev_live) G2B_HIP(c, hipEventSynchronize(c->home_ev));
  // streamed positions of each sequence ([0, pos)), and their total per layer
  int64_t per_layer = 0;
  for (int32_t i = 0; i < n_seq; i++) per_layer += (int64_t)c->h_seqs[i].pos;
  const int64_t extra = grid - n_units;
  int64_t g = 0;
  for (int64_t u = 0; u < n_units; u++) c->home_h[g++] = (int32_t)u;  // one each
  // the rest by cumulative rounding over the units' positions (u = li*n_seq + seq)
  int64_t cum = 0, given = 0;
  for (int64_t u = 0; u < n_units && per_layer > 0; u++) {
    cum += (int64_t)c->h_seqs[u % n_seq].pos;
    const int64_t upto = (int64_t)((__int128)extra * cum / ((__int128)per_layer * n_layers));
    for (; given < upto; given++) c->home_h[g++] = (int32_t)u;
  }
  for (; g < grid; g++) c->home_h[g] = (int32_t)(g % n_units);
  G2B_HIP(c, hipMemcpyAsync(c->home_d, c->home_h, (size_t)grid * sizeof(int32_t),
                            hipMemcpyHostToDevice, c->stream));
  G2B_HIP(c, hipEventRecord(c->home_ev, c->stream));
  c->home_ev_live = true;
  c->home_key[0] = c->batch_gen;
  c->home_key[1] = (uint64_t)n_layers;
  c->home_key[2] = (uint64_t)grid;
  *out = c->home_d;
  return G2B_OK;
}

// fixed: nullptr, or device memory of fixed_floats floats that holds this
// call's partials (and rotated q) - then nothing is allocated: no work queue,
// the RoPE table must already cover the positions, and the splits are
// lengthened until the partials fit.
int run_layers(g2b_ctx *c, const SeqDev *d_seqs, const SeqDev &one, int32_t n_seq,
               int32_t max_pos, int64_t total_pos, int32_t layer0, int32_t n_layers, float *q,
               const float *k, const float *v, float *att, int32_t att_stride,
               bool dry = false, float *fixed = nullptr, size_t fixed_floats = 0) {
  if (layer0 < 0 || n_layers < 1 || layer0 + n_layers > c->shape.n_layers)
    return fail(c, G2B_EINVAL, "layers [%d,%d) outside [0,%d)", layer0, layer0 + n_layers,
                c->shape.n_layers);
  if (!q || !k || !v) return fail(c, G2B_EINVAL, "q/k/v must be device pointers");
  if (att && att_stride < max_pos + 1)
    return fail(c, G2B_EINVAL, "att_stride %d < pos+1 = %d", att_stride, max_pos + 1);
  if (fixed) {
    if (c->sh.rope_on && c->rope_len < max_pos + 1)
      return fail(c, G2B_EINVAL, "the RoPE table covers %d positions, pos %d needs more: "
                  "allocate the KV with g2b_kv_alloc first", c->rope_len, max_pos);
  } else if (int rc = ensure_rope(c, max_pos + 1)) {
    return rc;
  }

  const int32_t nh = c->shape.n_heads, hd = c->shape.head_dim;
  const size_t nq = (size_t)nh * hd;
  // (k_layer reads q, k and v as 16-byte pieces; other pointers take the
  // generic kernels)
  const bool fast = decode_fast_available(c->sh) &&
                    (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15u) == 0;

  DecodeParams dp{};
  dp.sh = c->sh;
  dp.seqs = d_seqs;
  dp.one = one;
  dp.n_seq = n_seq;
  dp.layer0 = layer0;
  dp.q_rot = c->qrot;
  dp.q_out = q;
  dp.q_in = q;
  dp.k_in = k;
  dp.v_in = v;
  dp.rope = c->rope;
  dp.norm = norm_of(c);
  dp.att = att;
  dp.att_stride = att_stride;
  dp.qscale = c->qscale;
  dp.stamps = c->stamps ? c->stamps + (size_t)(c->stamp_next++ % c->stamp_launches) * 2 *
                                           c->stamp_cap * kStampWords
                        : nullptr;
  dp.stamp_cap = c->stamp_cap;
  // half-block lanes need twice the lanes per position; keep them only where they fit
  dp.tune_chunk = (c->tune_chunk == 16 && c->shape.kv_q8 &&
                   c->shape.n_kv_heads * (c->shape.head_dim / 16) <= 64) ? 16 : 0;
  // Staging pays for Q8_0 rows, whose per-lane block windows overlap, and
  // for F32 rows in calls over several layers (staged F32 rows lie
  // transposed in LDS; c3 all layers 601 against 720 us, c1 85.4 against
  // 94.9) and for one layer of a batch of F32 rows once its splits are sized
  // for it (below; c3 layer-serial 895-899 against 1067 us for per-lane
  // loads).  One layer of one sequence is bound by latency, not bytes:
  // per-lane loads, whose first trip is in flight during the setup (c2, 8193
  // positions: 545 us per layer-serial step against 580 us for staged
  // chunks).
  const bool one_unit = n_seq == 1 && n_layers == 1;
  dp.stage_mode = c->tune_stage < 0   ? 0
                  : c->tune_stage > 0 ? c->tune_stage
                  : one_unit          ? 0
                                      : kDefaultStageMode;
  dp.stage_rows = fast ? decode_stage_rows(c->sh, dp.tune_chunk, dp.stage_mode) : 0;
  if (dp.stage_rows == 0) dp.stage_mode = 0;
  dp.n_layers_call = n_layers;

  // split partials per sequence and layer: at most 512 (k_combine stages a
  // weight per partial), and n_seq of them within g2b_splits_per_layer_cap,
  // the bound g2b_hbm_bytes budgets
  int32_t splits_per_seq =
      (int32_t)std::min<uint64_t>(512, g2b_splits_per_layer_cap(n_seq) / (uint64_t)n_seq);
  // the fixed scratch: k_short's span counters (kFixedCtrInts, kept zero),
  // the rotated q (generic path), then the partials
  const size_t fixed_ctr = fixed ? kFixedCtrInts : 0;
  const size_t fixed_qrot = fixed && !fast ? ((size_t)n_layers * n_seq * nq + 63) & ~(size_t)63 : 0;
  if (fixed) {
    const size_t per_split = (size_t)n_layers * n_seq * nh * (size_t)(kPartHead + hd);
    const size_t used = fixed_ctr + fixed_qrot;
    const size_t fit = fixed_floats > used ? (fixed_floats - used) / per_split : 0;
    if (fit < 1)
      return fail(c, G2B_EUNSUP, "one split's partials (%zu bytes) exceed the %zu-byte scratch",
                  (used + per_split) * 4, fixed_floats * 4);
    splits_per_seq = (int32_t)std::min<size_t>((size_t)splits_per_seq, fit);
  }

  // k_short, no weights output: one workgroup per (KV head, span of
  // kShortMaxPos positions, sequence, layer).  Below kShortMaxPos positions
  // it is a single span that writes the output over q itself.  Longer
  // contexts take it (spans that merge their partials in the kernel, no
  // combine launch) only when g2b_ctx_tune_kernel(3) asks for it: one layer
  // of one sequence runs faster on k_layer's short static splits and the
  // one-round combine (c1, 17 spans x 8 KV heads = 136 workgroups: 525.9 us
  // per layer-serial step against 459 us; c2, 65 x 8 = 520: 822 against
  // 545; all 28 layers in one call 108.7 against 92.7 us).  An explicit
  // split length or work-queue piece (g2b_ctx_tune) keeps the split kernels.
  const int32_t n_spans = max_pos / kShortMaxPos + 1;
  const bool short_ok = fast && !att && c->split_override == 0 && c->tune_piece == 0 &&
                        short_available(c->sh);
  const bool spans_wanted = c->tune_kernel == 3;
  const bool spans_fit = n_spans <= std::min<int32_t>(kShortMaxSpans, splits_per_seq) &&
                         (!fixed || (size_t)n_layers * n_seq * c->shape.n_kv_heads <= fixed_ctr);
  if (short_ok && (n_spans == 1 || (spans_wanted && spans_fit))) {
    dp.max_splits = n_spans;
    dp.span_ctr = nullptr;
    if (n_spans > 1) {
      const size_t ctrs = (size_t)n_layers * n_seq * c->shape.n_kv_heads;
      if (fixed) {
        dp.span_ctr = reinterpret_cast<int32_t *>(fixed);
        dp.part = fixed + fixed_ctr;
      } else {
        const size_t part_floats = (size_t)n_layers * n_seq * nh * (size_t)n_spans *
                                   (size_t)(kPartHead + hd);
        const size_t part_limit = (size_t)c->shape.n_layers *
                                  (size_t)g2b_splits_per_layer_cap(n_seq) * nh *
                                  (size_t)(kPartHead + hd);
        if (int rc = grow(c, &c->part, &c->part_cap, part_floats, part_limit)) return rc;
        if (int rc = span_counters(c, ctrs)) return rc;
        dp.span_ctr = c->span_ctr;
        dp.part = c->part;
      }
    }
    if (dry) return G2B_OK;
    set_sched(c, G2B_KERNEL_SHORT, kShortMaxPos, 0, n_spans,
              (int64_t)c->shape.n_kv_heads * n_spans * n_seq * n_layers, true);
    hipEvent_t ev1 = nullptr;
    if (int rc = prof_begin(c, &ev1)) return rc;
    G2B_HIP(c, launch_short(dp, n_layers, c->stream));
    if (ev1) G2B_HIP(c, hipEventRecord(ev1, c->stream));
    return G2B_OK;
  }

  // k_tiles (K scores on the matrix cores) for Q8_0 KV with wide GQA groups,
  // no weights output; it stages tiles of kTilesRows positions per
  // workgroup, so pieces and splits are multiples of that.
  const bool tiles = fast && !att && c->tune_kernel != 1 && c->tune_chunk == 0 &&
                     (c->tune_stage == 0 || c->tune_stage == 2) && tiles_available(c->sh);
  if (tiles) {
    dp.stage_mode = 2;
    dp.stage_rows = kTilesRows;
  }

  // Work queue (staged streaming) when few enough waves share each unit's
  // counters - with more units (sequence, layer) than resident workgroups,
  // the workgroups take the units in turn; otherwise static splits, sized
  // so the launch's workgroups form whole rounds.
  const int64_t n_units = (int64_t)n_seq * n_layers;
  // k_layer's work queue pulls its chunks straight into LDS (mode 1): 1-2%
  // faster than register staging on the batched configs, while a single
  // sequence's static splits, bound by latency, keep register staging.  The
  // work queue's slots are counted for the variant it would run (the
  // register-staging variant holds more registers: fewer resident
  // workgroups, which had sent c2's all-layers call through the work queue,
  // 115 against 97-101 us).
  DecodeParams wq_dp = dp;
  if (!tiles && c->tune_stage == 0 && dp.stage_mode == kDefaultStageMode) {
    const int32_t r1 = decode_stage_rows(c->sh, dp.tune_chunk, 1);
    if (r1 > 0) {
      wq_dp.stage_mode = 1;
      wq_dp.stage_rows = r1;
    }
  }
  const int64_t wq_slots = tiles                           ? tiles_slots(c, true)
                           : fast && wq_dp.stage_mode != 0 ? slots_for(c, wq_dp, true)
                                                            : 0;
  // (F32 rows: static splits unless a piece is asked for - c3 all layers
  // 601 us static against 659 us through the work queue)
  const bool use_wq = !fixed && fast && dp.stage_mode != 0 && c->tune_piece >= 0 &&
                      (c->tune_piece > 0 ||
                       (c->shape.kv_q8 && wq_slots * kWavesPerSplit <= n_units * kWqMaxWavesPerUnit));
  if (use_wq && !tiles) {
    dp.stage_mode = wq_dp.stage_mode;
    dp.stage_rows = wq_dp.stage_rows;
  }
  const int64_t slots = use_wq ? (tiles ? wq_slots : slots_for(c, dp, true))
                        : tiles ? tiles_slots(c, false)
                                : slots_for(c, dp, false);
  int32_t max_splits;
  if (use_wq) {
    const int64_t wq_lines = n_units + 1;  // the units and the next-unit counter
    if (wq_lines > c->wq_cap) {
      G2B_HIP(c, hipStreamSynchronize(c->stream));
      if (c->wq) G2B_HIP(c, hipFree(c->wq));
      c->wq = nullptr;
      c->wq_cap = 0;
      const int32_t cap = (int32_t)std::max<int64_t>(wq_lines, G2B_WQ_MIN_LINES);
      const size_t bytes = (size_t)2 * cap * kWqStride * sizeof(int32_t);
      if (hipMalloc((void **)&c->wq, bytes) != hipSuccess) {
        c->wq = nullptr;
        (void)hipGetLastError();
        return fail(c, G2B_ENOMEM, "work-queue counters");
      }
      c->wq_cap = cap;
      c->wq_reset = true;
    }
    if (c->wq_reset) {
      G2B_HIP(c, hipMemsetAsync(c->wq, 0, (size_t)2 * c->wq_cap * kWqStride * sizeof(int32_t),
                                c->stream));
      c->wq_set = 0;
      c->wq_dirty[0] = c->wq_dirty[1] = 0;
      c->wq_reset = false;
    }
    max_splits = (int32_t)std::min<int64_t>(
        std::max<int64_t>(kWqMinParts, (slots + n_units - 1) / n_units + 8),
        std::min<int64_t>(2048, splits_per_seq));
    const int32_t R = dp.stage_rows;
    const int64_t streamed = (total_pos - n_seq) * (int64_t)n_layers;  // positions [0, pos)
    // (automatic: about kWqClaimsPerWave claims per wave of the grid; with
    // more units than workgroups also at most 1/kWqUnitPieces of an average
    // unit, so that a workgroup that has a unit to itself keeps its four
    // waves evenly loaded)
    int64_t pl = streamed / (slots * kWavesPerSplit * kWqClaimsPerWave);
    if (n_units > slots) pl = std::min<int64_t>(pl, streamed / (n_units * kWqUnitPieces));
    if (c->tune_piece > 0) pl = c->tune_piece;
    pl = std::min<int64_t>(std::max<int64_t>(pl, R), (int64_t)64 * R);
    dp.piece_len = (int32_t)(pl - pl % R);
    dp.piece_big = dp.piece_len * kWqBigFactor;
    dp.wq = c->wq;
    dp.wq_set = c->wq_set;
    dp.wq_cap = c->wq_cap;
    dp.wq_zero_units = c->wq_dirty[c->wq_set ^ 1];
    dp.wq_grid = (int32_t)slots;
    dp.split_len = 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    G2B_HIP(c, hipStreamIsCapturing(c->stream, &cap));
    // (not under capture: a replay would copy whatever the staging holds then)
    if (d_seqs && d_seqs == c->d_seqs && c->h_seqs && cap == hipStreamCaptureStatusNone)
      if (int rc = wq_home_table(c, n_seq, n_layers, slots, &dp.home)) return rc;
  } else {
    // (measured: four staged chunks or eight per-lane wave-steps per wave, four
    // for one layer of one sequence)
    const int32_t ppw = decode_ppw(c->sh, dp.tune_chunk);
    const int32_t min_len = !fast                ? 64
                            : tiles             ? 8 * kTilesRows
                            : dp.stage_rows > 0 ? kWavesPerSplit * 4 * dp.stage_rows
                            : one_unit          ? kWavesPerSplit * 4 * ppw
                                                : kWavesPerSplit * 8 * ppw;
    // Per-lane loads (stage_rows == 0): for one sequence a round is one
    // workgroup per CU (c1 all layers: 252 workgroups of 228 positions
    // 92.7 us, 364 of 161 positions 109 us), and one layer of it takes half
    // of that (fewer partials for the combine; c1, 2049 positions: 459 us per
    // layer-serial step at 129 splits, 487 at 147, 507 at 171 and 522 at 228;
    // c2, 8193 positions: 545 at 129, 561 at 249); for batches ~0.7 of the
    // resident workgroups - measured on the 64-sequence SmolLM2 F32 batch
    // (c3): 1304 us per layer-serial step at 0.72 of a round against 1490 us
    // at 0.9, 1559 us at 1.13 and 1458 us at 1.5 rounds
    // Staged F32 rows of one sequence count one workgroup per CU as a round
    // too (c1 all layers: 252 workgroups 83.3 us, 504 84.3-85.9 us).
    // Staged F32 rows of one layer of a batch: about 0.78 of the resident
    // workgroups, counting half a split per sequence for the ragged ends (c3,
    // 64 sequences, 73527 positions, 512 slots: 405 workgroups of 201
    // positions; layer-serial 895 us at 405-414 workgroups, 913-922 at
    // 363-387, 1127-1173 at 428-492, 948-990 at 286-319).
    const int64_t f32_batch_slots =
        std::max<int64_t>(slots / 8, slots * 78 / 100 - (int64_t)n_seq / 2);
    const int64_t split_slots = !fast ? slots
                                : dp.stage_rows > 0
                                    ? (c->shape.kv_q8  ? slots
                                       : n_seq == 1    ? std::max(1, c->n_cu)
                                       : n_layers == 1 ? f32_batch_slots
                                                       : slots)
                                : one_unit   ? std::max(1, c->n_cu / 2)
                                : n_seq == 1 ? std::max(1, c->n_cu)
                                             : slots * 7 / 10;
    int32_t split_len = choose_split(c, std::max<int64_t>(split_slots, 1), n_seq, total_pos,
                                     max_pos, n_layers, fast, min_len);
    if (fast && one_unit && dp.stage_rows == 0 && c->split_override == 0) {
      // whole trips (two wave-steps) for every wave: a wave with one more
      // trip than the others waits one more round trip (c1: 489 us per
      // layer-serial step at 17 positions per split, 459 at 16)
      const int32_t trip = kWavesPerSplit * 2 * ppw;
      split_len = std::max(min_len, split_len / trip * trip);
    }
    max_splits = (max_pos + 1 + split_len - 1) / split_len;
    if (max_splits > splits_per_seq) {  // lengthen the splits to stay within the budget
      split_len = (int32_t)(((int64_t)max_pos + splits_per_seq) / splits_per_seq);
      max_splits = (max_pos + 1 + split_len - 1) / split_len;
    }
    if (!fast && split_len > kGenericMaxSplit)
      return fail(c, G2B_EUNSUP, "context %d of %d sequences needs splits of %d positions "
                  "(> %d on the generic kernel)", max_pos + 1, n_seq, split_len, kGenericMaxSplit);
    dp.split_len = split_len;
  }
  dp.max_splits = max_splits;
  // one split per unit: the decode kernel writes the output, no combine
  const bool direct = fast && !use_wq && max_splits == 1 && !att;
  dp.direct_out = direct ? 1 : 0;


  const size_t part_floats = (size_t)n_layers * n_seq * nh * (size_t)max_splits *
                             (size_t)(kPartHead + hd);
  if (fixed) {
    dp.q_rot = fixed + fixed_ctr;
    dp.part = fixed + fixed_ctr + fixed_qrot;
  } else {
    const size_t part_limit = (size_t)c->shape.n_layers *
                              (size_t)g2b_splits_per_layer_cap(n_seq) * nh *
                              (size_t)(kPartHead + hd);
    if (int rc = grow(c, &c->part, &c->part_cap, part_floats, part_limit)) return rc;
    if (!fast) {
      const size_t qf = (size_t)n_layers * n_seq * nq;
      if (int rc = grow(c, &c->qrot, &c->qrot_cap, qf, qf)) return rc;
    }
    dp.part = c->part;
    dp.q_rot = c->qrot;
  }
  if (dry) return G2B_OK;  // (the buffers this schedule needs exist now)

  if (!fast) {  // generic shapes: append, decode, combine
    AppendParams ap{};
    ap.sh = c->sh;
    ap.seqs = d_seqs;
    ap.one = one;
    ap.n_seq = n_seq;
    ap.layer0 = layer0;
    ap.q_in = q;
    ap.q_rot = fixed ? fixed + fixed_ctr : c->qrot;
    ap.k_in = k;
    ap.v_in = v;
    ap.rope = c->rope;
    ap.norm = norm_of(c);
    G2B_HIP(c, launch_append_batch(ap, n_layers, c->stream));
  }
  int used_fast = 0;
  hipEvent_t ev1 = nullptr;
  if (int rc = prof_begin(c, &ev1)) return rc;
  if (use_wq) c->wq_reset = true;  // until both launches below are queued
  if (tiles) {
    used_fast = 1;
    G2B_HIP(c, launch_tiles(dp, n_layers, c->stream));
  } else {
    G2B_HIP(c, launch_decode(dp, n_layers, c->stream, fast, &used_fast));
  }
  // (what launch_layer instantiates: staging only with whole 16-byte row
  // pieces; k_tiles always pulls its tiles into LDS by DMA)
  const int32_t staging = tiles ? 1 : used_fast && dp.stage_rows > 0 ? dp.stage_mode : 0;
  set_sched(c, tiles ? G2B_KERNEL_TILES : used_fast ? G2B_KERNEL_LAYER : G2B_KERNEL_GENERIC,
            dp.split_len, use_wq ? dp.piece_len : 0, max_splits,
            use_wq ? slots : (int64_t)max_splits * n_seq * n_layers, direct && used_fast,
            staging, used_fast && !tiles ? decode_chunk(c->sh, dp.tune_chunk) : 0, att != nullptr);
  if (ev1) G2B_HIP(c, hipEventRecord(ev1, c->stream));
  if (!direct || !used_fast) G2B_HIP(c, launch_combine(dp, n_layers, c->stream));
  if (use_wq) {
    // this launch dirtied its set; the combine zeroed the other one
    c->wq_dirty[c->wq_set] = std::max<int32_t>(c->wq_dirty[c->wq_set], (int32_t)n_units + 1);
    c->wq_dirty[c->wq_set ^ 1] = 0;
    c->wq_set ^= 1;
    c->wq_reset = false;
  }
  return G2B_OK;
}

}  // namespace

// Decode attention of one sequence whose descriptor lives in device memory
// (the kernels read pos from it), scheduled for any pos <= max_pos: the
// launches stay valid from step to step, as a captured step graph needs.
int g2b::attn_forward_device_seq(g2b_ctx *c, int32_t layer, const SeqDev *d_seq,
                                 int32_t max_pos, float *q, const float *k, const float *v) {
  if (!c || !d_seq) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  SeqDev none{};
  return run_layers(c, d_seq, none, 1, max_pos, (int64_t)max_pos + 1, layer, 1, q, k, v, nullptr,
                    0);
}

int g2b::attn_reserve_device_seq(g2b_ctx *c, int32_t max_pos, float *q, const float *k,
                                 const float *v) {
  if (!c) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  SeqDev none{};
  return run_layers(c, nullptr, none, 1, max_pos, (int64_t)max_pos + 1, 0, 1, q, k, v, nullptr, 0,
                    true);
}

extern "C" {

const char *g2b_strerror(int32_t code) {
  switch (code) {
    case G2B_OK: return "ok";
    case G2B_EINVAL: return "invalid argument";
    case G2B_EPOS: return "position outside [0, ctx)";
    case G2B_ENOKV: return "KV cache not allocated";
    case G2B_ENOMEM: return "device allocation failed";
    case G2B_EDEVICE: return "HIP runtime error";
    case G2B_ESWAP: return "file-backed KV cannot live in HBM";
    case G2B_EUNSUP: return "unsupported shape";
    default: return "unknown error";
  }
}

const char *g2b_ctx_last_error(g2b_ctx *c) { return c ? c->err.c_str() : ""; }

size_t g2b_kv_row_bytes(const g2b_shape *s) { return s ? row_bytes_of(s) : 0; }

uint64_t g2b_kv_bytes(const g2b_shape *s, int32_t ctx_cap) {
  if (!s || ctx_cap <= 0 || s->n_layers <= 0) return 0;
  return (uint64_t)s->n_layers * (uint64_t)ctx_cap * (uint64_t)row_bytes_of(s);
}

uint64_t g2b_kv_offset(const g2b_shape *s, int32_t ctx_cap, int32_t layer, int32_t pos) {
  if (!s) return 0;
  return ((uint64_t)layer * (uint64_t)ctx_cap + (uint64_t)pos) * (uint64_t)row_bytes_of(s);
}

int g2b_ctx_create(g2b_ctx **out, int32_t device, const g2b_shape *s) {
  if (!out || !s) return G2B_EINVAL;
  *out = nullptr;
  if (s->n_layers < 1 || s->n_heads < 1 || s->n_kv_heads < 1 || s->head_dim < 2 ||
      (s->head_dim & 1) || s->n_heads % s->n_kv_heads)
    return G2B_EINVAL;
  if ((int64_t)s->n_kv_heads * s->head_dim + s->n_heads > 16384) return G2B_EUNSUP;  // append LDS
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
    (void)hipGetLastError();
    return G2B_EDEVICE;
  }
  g2b_ctx *c = new (std::nothrow) g2b_ctx();
  if (!c) return G2B_ENOMEM;
  c->device = device;
  c->shape = *s;
  c->sh.n_layers = s->n_layers;
  c->sh.n_heads = s->n_heads;
  c->sh.n_kv_heads = s->n_kv_heads;
  c->sh.head_dim = s->head_dim;
  c->sh.arch_llama = s->arch == G2B_ARCH_LLAMA ? 1 : 0;
  c->sh.kv_q8 = s->kv_q8 ? 1 : 0;
  c->sh.rope_on = (s->head_dim / 2) <= 512 ? 1 : 0;
  c->sh.row_bytes = (uint32_t)row_bytes_of(s);
  // l5_model.c:518 scale, times log2(e) for exp2-based softmax
  c->qscale = (1.f / sqrtf((float)s->head_dim)) * 1.44269504088896340736f;
  if (hipSetDevice(device) != hipSuccess ||
      hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&c->seqs_ev, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    if (c->own) (void)hipStreamDestroy(c->own);
    delete c;
    return G2B_EDEVICE;
  }
  c->stream = c->own;
  if (fixed_scratch_of(device, &c->fixed) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipEventDestroy(c->seqs_ev);
    (void)hipStreamDestroy(c->own);
    delete c;
    return G2B_EDEVICE;
  }
  int n_cu = 0;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    n_cu = 0;
  (void)hipGetLastError();
  c->n_cu = std::max(1, n_cu);
  memset(c->occ_cache, 0, sizeof c->occ_cache);
  *out = c;
  return G2B_OK;
}

int g2b_ctx_destroy(g2b_ctx *c) {
  if (!c) return G2B_EINVAL;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  if (c->own) (void)hipStreamSynchronize(c->own);
  if (c->rope) (void)hipFree(c->rope);
  if (c->d_seqs) (void)hipFree(c->d_seqs);
  if (c->h_seqs) (void)hipHostFree(c->h_seqs);
  if (c->qrot) (void)hipFree(c->qrot);
  if (c->part) (void)hipFree(c->part);
  if (c->stamps) (void)hipFree(c->stamps);
  if (c->hstage) (void)hipFree(c->hstage);
  if (c->qkn_w) (void)hipFree(c->qkn_w);
  if (c->qkn_on) (void)hipFree(c->qkn_on);
  if (c->wq) (void)hipFree(c->wq);
  if (c->span_ctr) (void)hipFree(c->span_ctr);
  if (c->home_d) (void)hipFree(c->home_d);
  if (c->home_h) (void)hipHostFree(c->home_h);
  if (c->home_ev) (void)hipEventDestroy(c->home_ev);
  if (c->seqs_ev) (void)hipEventDestroy(c->seqs_ev);
  for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
  if (c->own) (void)hipStreamDestroy(c->own);
  delete c;
  return G2B_OK;
}

int g2b_ctx_set_stream(g2b_ctx *c, void *stream) {
  if (!c) return G2B_EINVAL;
  c->stream = stream ? (hipStream_t)stream : c->own;
  return G2B_OK;
}

void *g2b_ctx_stream(g2b_ctx *c) { return c ? (void *)c->stream : nullptr; }

int g2b_kv_alloc(g2b_ctx *c, int32_t ctx_cap, void **kc, void **vc) {
  if (!c || !kc || !vc || ctx_cap < 1) return fail(c, G2B_EINVAL, "bad kv_alloc arguments");
  *kc = *vc = nullptr;
  if (int rc = set_device(c)) return rc;
  const size_t bytes = (size_t)g2b_kv_bytes(&c->shape, ctx_cap) + kKvSlack;
  void *k = nullptr, *v = nullptr;
  if (hipMalloc(&k, bytes) != hipSuccess || hipMalloc(&v, bytes) != hipSuccess) {
    (void)hipGetLastError();
    if (k) (void)hipFree(k);
    return fail(c, G2B_ENOMEM, "KV allocation of 2 x %zu bytes failed", bytes);
  }
  if (zero_device(c, k, bytes) != G2B_OK || zero_device(c, v, bytes) != G2B_OK) {
    (void)hipFree(k);
    (void)hipFree(v);
    return fail(c, G2B_EDEVICE, "KV memset failed");
  }
  if (int rc = ensure_rope(c, ctx_cap)) {
    (void)hipFree(k);
    (void)hipFree(v);
    return rc;
  }
  *kc = k;
  *vc = v;
  return G2B_OK;
}

int g2b_kv_free(g2b_ctx *c, void *kc, void *vc) {
  if (!c) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  if (kc) G2B_HIP(c, hipFree(kc));
  if (vc) G2B_HIP(c, hipFree(vc));
  return G2B_OK;
}

int g2b_kv_read(g2b_ctx *c, const void *cache, uint64_t offset, uint64_t nbytes, void *host) {
  if (!c) return G2B_EINVAL;
  if (!cache) return fail(c, G2B_ENOKV, "KV cache not allocated");
  if (!host && nbytes) return fail(c, G2B_EINVAL, "null host buffer");
  if (nbytes == 0) return G2B_OK;
  if (int rc = set_device(c)) return rc;
  G2B_HIP(c, hipMemcpyAsync(host, (const uint8_t *)cache + offset, (size_t)nbytes,
                            hipMemcpyDeviceToHost, c->stream));
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  return G2B_OK;
}

int g2b_kv_append_rows(g2b_ctx *c, void *kc, void *vc, int32_t ctx_cap, int32_t layer,
                       int32_t pos0, int32_t n_rows, const float *k, const float *v) {
  if (!c) return G2B_EINVAL;
  if (!kc || !vc) return fail(c, G2B_ENOKV, "KV cache not allocated");
  if (!k || !v || n_rows < 0 || layer < 0 || layer >= c->shape.n_layers)
    return fail(c, G2B_EINVAL, "bad append_rows arguments");
  if (pos0 < 0 || (int64_t)pos0 + n_rows > ctx_cap)
    return fail(c, G2B_EPOS, "rows [%d,%d) outside [0,%d)", pos0, pos0 + n_rows, ctx_cap);
  if (n_rows == 0) return G2B_OK;
  if (int rc = set_device(c)) return rc;
  if (int rc = ensure_rope(c, pos0 + n_rows)) return rc;
  AppendParams ap{};
  ap.sh = c->sh;
  ap.seqs = nullptr;
  ap.one.pos = pos0;
  ap.one.ctx_cap = ctx_cap;
  ap.one.k = (uint8_t *)kc;
  ap.one.v = (uint8_t *)vc;
  ap.n_seq = 1;
  ap.k_in = k;
  ap.v_in = v;
  ap.rope = c->rope;
  ap.norm = norm_of(c);
  ap.pos0 = pos0;
  G2B_HIP(c, launch_append_rows(ap, layer, n_rows, c->stream));
  return G2B_OK;
}

int g2b_set_qk_norm(g2b_ctx *c, int32_t layer, const float *q_norm, const float *k_norm,
                    float eps) {
  if (!c) return G2B_EINVAL;
  if (layer < 0 || layer >= c->shape.n_layers)
    return fail(c, G2B_EINVAL, "layer %d outside [0,%d)", layer, c->shape.n_layers);
  const int32_t L = c->shape.n_layers, hd = c->shape.head_dim;
  bool others = false;
  for (int32_t i = 0; i < (int32_t)c->qkn_on_h.size(); i++) others |= i != layer && c->qkn_on_h[i];
  if (others && memcmp(&eps, &c->qkn_eps, sizeof eps) != 0)
    return fail(c, G2B_EINVAL, "eps %g differs from %g set for other layers (one per model)",
                (double)eps, (double)c->qkn_eps);
  if (int rc = set_device(c)) return rc;
  if (!c->qkn_w) {
    if (hipMalloc((void **)&c->qkn_w, (size_t)L * 2 * hd * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&c->qkn_on, (size_t)L * sizeof(int32_t)) != hipSuccess) {
      (void)hipGetLastError();
      if (c->qkn_w) (void)hipFree(c->qkn_w);
      c->qkn_w = nullptr;
      return fail(c, G2B_ENOMEM, "QK-norm weights");
    }
    c->qkn_on_h.assign((size_t)L, 0);
    if (int rc = zero_device(c, c->qkn_on, (size_t)L * sizeof(int32_t))) return rc;
  }
  // Calls already queued may read the weights: let them finish first.
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  float *wl = c->qkn_w + (size_t)layer * 2 * hd;
  if (q_norm) G2B_HIP(c, hipMemcpy(wl, q_norm, (size_t)hd * sizeof(float), hipMemcpyHostToDevice));
  if (k_norm)
    G2B_HIP(c, hipMemcpy(wl + hd, k_norm, (size_t)hd * sizeof(float), hipMemcpyHostToDevice));
  const int32_t on = (q_norm ? 1 : 0) | (k_norm ? 2 : 0);
  G2B_HIP(c, hipMemcpy(c->qkn_on + layer, &on, sizeof on, hipMemcpyHostToDevice));
  c->qkn_on_h[(size_t)layer] = on;
  c->qkn_eps = eps;
  return G2B_OK;
}

int g2b_batch_begin(g2b_ctx *c, int32_t n_seq, const g2b_seq *seqs) {
  if (!c) return G2B_EINVAL;
  if (n_seq < 1 || !seqs) return fail(c, G2B_EINVAL, "empty batch");
  if (n_seq > 65535) return fail(c, G2B_EUNSUP, "batch of %d sequences", n_seq);
  int32_t max_pos = 0;
  int64_t total = 0;
  for (int32_t i = 0; i < n_seq; i++) {
    const g2b_seq &s = seqs[i];
    if (!s.kcache || !s.vcache) return fail(c, G2B_ENOKV, "sequence %d has no KV", i);
    if (misaligned(s.kcache) || misaligned(s.vcache))
      return fail(c, G2B_EINVAL, "sequence %d: KV caches must be 16-byte aligned", i);
    if (s.ctx_cap < 1 || s.pos < 0 || s.pos >= s.ctx_cap)
      return fail(c, G2B_EPOS, "sequence %d: pos=%d outside [0,%d)", i, s.pos, s.ctx_cap);
    max_pos = std::max(max_pos, s.pos);
    total += (int64_t)s.pos + 1;
  }
  if (int rc = set_device(c)) return rc;
  if (n_seq > c->seqs_cap) {
    G2B_HIP(c, hipStreamSynchronize(c->stream));
    if (c->d_seqs) G2B_HIP(c, hipFree(c->d_seqs));
    if (c->h_seqs) G2B_HIP(c, hipHostFree(c->h_seqs));
    c->d_seqs = nullptr;
    c->h_seqs = nullptr;
    c->seqs_cap = 0;
    c->seqs_ev_live = false;
    const int32_t cap = std::max<int32_t>(n_seq, (int32_t)G2B_SEQ_DESC_MIN);
    if (hipMalloc((void **)&c->d_seqs, cap * sizeof(SeqDev)) != hipSuccess ||
        hipHostMalloc((void **)&c->h_seqs, cap * sizeof(SeqDev), hipHostMallocDefault) !=
            hipSuccess) {
      (void)hipGetLastError();
      return fail(c, G2B_ENOMEM, "batch descriptors");
    }
    c->seqs_cap = cap;
  }
  if (c->seqs_ev_live) G2B_HIP(c, hipEventSynchronize(c->seqs_ev));
  for (int32_t i = 0; i < n_seq; i++) {
    SeqDev d{};
    d.pos = seqs[i].pos;
    d.ctx_cap = seqs[i].ctx_cap;
    d.k = (uint8_t *)seqs[i].kcache;
    d.v = (uint8_t *)seqs[i].vcache;
    c->h_seqs[i] = d;
    if (i == 0) c->seq0 = d;
  }
  G2B_HIP(c, hipMemcpyAsync(c->d_seqs, c->h_seqs, n_seq * sizeof(SeqDev),
                            hipMemcpyHostToDevice, c->stream));
  G2B_HIP(c, hipEventRecord(c->seqs_ev, c->stream));
  c->seqs_ev_live = true;
  if (int rc = ensure_rope(c, max_pos + 1)) return rc;
  c->n_seq = n_seq;
  c->max_pos = max_pos;
  c->total_pos = total;
  c->batch_gen++;
  return G2B_OK;
}

int g2b_attn_layers(g2b_ctx *c, int32_t layer0, int32_t n_layers, float *q, const float *k,
                    const float *v, float *att, int32_t att_stride) {
  if (!c) return G2B_EINVAL;
  if (c->n_seq < 1) return fail(c, G2B_EINVAL, "no batch: call g2b_batch_begin first");
  if (int rc = set_device(c)) return rc;
  // One sequence travels in the kernel arguments: no dependent load of its
  // descriptor at the start of every workgroup.
  SeqDev none{};
  if (c->n_seq == 1)
    return run_layers(c, nullptr, c->seq0, 1, c->max_pos, c->total_pos, layer0, n_layers, q, k,
                      v, att, att_stride);
  return run_layers(c, c->d_seqs, none, c->n_seq, c->max_pos, c->total_pos, layer0, n_layers,
                    q, k, v, att, att_stride);
}

int g2b_attn_forward(g2b_ctx *c, int32_t layer, int32_t pos, int32_t ctx_cap, void *kc,
                     void *vc, float *q, const float *k, const float *v, float *att) {
  if (!c) return G2B_EINVAL;
  if (!kc || !vc) return fail(c, G2B_ENOKV, "KV cache not allocated");
  if (misaligned(kc) || misaligned(vc))
    return fail(c, G2B_EINVAL, "KV caches must be 16-byte aligned");
  if (ctx_cap < 1 || pos < 0 || pos >= ctx_cap)
    return fail(c, G2B_EPOS, "pos=%d outside [0,%d)", pos, ctx_cap);
  if (int rc = set_device(c)) return rc;
  SeqDev one{};
  one.pos = pos;
  one.ctx_cap = ctx_cap;
  one.k = (uint8_t *)kc;
  one.v = (uint8_t *)vc;
  return run_layers(c, nullptr, one, 1, pos, (int64_t)pos + 1, layer, 1, q, k, v, att, ctx_cap);
}

int g2b_attn_forward_noalloc(g2b_ctx *c, int32_t layer, int32_t pos, int32_t ctx_cap, void *kc,
                             void *vc, float *q, const float *k, const float *v) {
  if (!c) return G2B_EINVAL;
  if (!kc || !vc) return fail(c, G2B_ENOKV, "KV cache not allocated");
  if (misaligned(kc) || misaligned(vc))
    return fail(c, G2B_EINVAL, "KV caches must be 16-byte aligned");
  if (ctx_cap < 1 || pos < 0 || pos >= ctx_cap)
    return fail(c, G2B_EPOS, "pos=%d outside [0,%d)", pos, ctx_cap);
  if (!c->fixed) return fail(c, G2B_EDEVICE, "no scratch address for device %d", c->device);
  if (int rc = set_device(c)) return rc;
  SeqDev one{};
  one.pos = pos;
  one.ctx_cap = ctx_cap;
  one.k = (uint8_t *)kc;
  one.v = (uint8_t *)vc;
  return run_layers(c, nullptr, one, 1, pos, (int64_t)pos + 1, layer, 1, q, k, v, nullptr, 0,
                    false, c->fixed, kFixedScratchBytes / sizeof(float));
}

int g2b_attn_forward_host(g2b_ctx *c, int32_t layer, int32_t pos, int32_t ctx_cap, void *kc,
                          void *vc, float *q, const float *k, const float *v, float *att) {
  if (!c) return G2B_EINVAL;
  if (!q || !k || !v) return fail(c, G2B_EINVAL, "q/k/v must be host pointers");
  if (!kc || !vc) return fail(c, G2B_ENOKV, "KV cache not allocated");
  if (misaligned(kc) || misaligned(vc))
    return fail(c, G2B_EINVAL, "KV caches must be 16-byte aligned");
  if (ctx_cap < 1 || pos < 0 || pos >= ctx_cap)
    return fail(c, G2B_EPOS, "pos=%d outside [0,%d)", pos, ctx_cap);
  if (int rc = set_device(c)) return rc;
  const size_t nq = (size_t)c->shape.n_heads * c->shape.head_dim;
  const size_t nkv = (size_t)c->shape.n_kv_heads * c->shape.head_dim;
  const size_t natt = att ? (size_t)c->shape.n_heads * (size_t)ctx_cap : 0;
  if (int rc = grow(c, &c->hstage, &c->hstage_cap, nq + 2 * nkv + natt, nq + 2 * nkv + natt))
    return rc;
  float *dq = c->hstage, *dk = dq + nq, *dv = dk + nkv, *da = att ? dv + nkv : nullptr;
  G2B_HIP(c, hipMemcpyAsync(dq, q, nq * 4, hipMemcpyHostToDevice, c->stream));
  G2B_HIP(c, hipMemcpyAsync(dk, k, nkv * 4, hipMemcpyHostToDevice, c->stream));
  G2B_HIP(c, hipMemcpyAsync(dv, v, nkv * 4, hipMemcpyHostToDevice, c->stream));
  if (int rc = g2b_attn_forward(c, layer, pos, ctx_cap, kc, vc, dq, dk, dv, da)) return rc;
  G2B_HIP(c, hipMemcpyAsync(q, dq, nq * 4, hipMemcpyDeviceToHost, c->stream));
  if (att)
    G2B_HIP(c, hipMemcpyAsync(att, da, natt * 4, hipMemcpyDeviceToHost, c->stream));
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  return G2B_OK;
}

int g2b_sync(g2b_ctx *c) {
  if (!c) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  return G2B_OK;
}

size_t g2b_matmul_row_bytes(int32_t type, int32_t n) {
  if (n < 0) return 0;
  switch (type) {
    case G2B_T_F32: return (size_t)n * 4u;
    case G2B_T_F16: return (size_t)n * 2u;
    case G2B_T_Q8_0: return (size_t)(n / 32) * 34u;
    case G2B_T_Q4_0: return (size_t)(n / 32) * 18u;
    case G2B_T_Q4_1: return (size_t)(n / 32) * 20u;
    default: return 0;
  }
}

int g2b_matmul(g2b_ctx *c, float *out, const float *x, const void *w, int32_t type, int32_t n,
               int32_t d) {
  if (!c) return G2B_EINVAL;
  if (type != G2B_T_F32 && type != G2B_T_F16 && type != G2B_T_Q8_0 && type != G2B_T_Q4_0 &&
      type != G2B_T_Q4_1)
    return fail(c, G2B_EUNSUP, "weight type %d has no device GEMV", type);
  if (int rc = set_device(c)) return rc;
  if (!out || !x || !w || n <= 0 || d <= 0) {  // matmul_q's guard (l2_codec.c:343-346)
    if (out && d > 0) G2B_HIP(c, launch_fill_zero(out, d, c->stream));
    return G2B_OK;
  }
  if (type == G2B_T_Q4_1 && n % 32)
    return fail(c, G2B_EINVAL, "Q4_1 rows must be whole blocks (n %% 32 == 0), n = %d", n);
  if (((uintptr_t)w & 1u) && type != G2B_T_F32)
    return fail(c, G2B_EINVAL, "F16 and quantised weights must be 2-byte aligned");
  if (((uintptr_t)w & 3u) && type == G2B_T_F32)
    return fail(c, G2B_EINVAL, "F32 weights must be 4-byte aligned");
  GemvParams p{};
  p.out = out;
  p.x = x;
  p.w = (const uint8_t *)w;
  p.n = n;
  p.d = d;
  p.x_vec4 = ((uintptr_t)x & 15u) == 0;
  G2B_HIP(c, launch_gemv(p, type, c->n_cu, c->stream));
  return G2B_OK;
}

int g2b_matmul_host(g2b_ctx *c, float *out, const float *x, const void *w, int32_t type,
                    int32_t n, int32_t d) {
  if (!c) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  if (!out || d <= 0) return g2b_matmul(c, nullptr, nullptr, nullptr, type, 0, 0);
  const size_t nx = (x && w && n > 0) ? (size_t)n : 0;
  if (int rc = grow(c, &c->hstage, &c->hstage_cap, nx + (size_t)d + 4, nx + (size_t)d + 4))
    return rc;
  float *dx = c->hstage, *dout = dx + ((nx + 3) & ~(size_t)3);
  if (nx) G2B_HIP(c, hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, c->stream));
  if (int rc = g2b_matmul(c, dout, nx ? dx : nullptr, w, type, n, d)) return rc;
  G2B_HIP(c, hipMemcpyAsync(out, dout, (size_t)d * 4, hipMemcpyDeviceToHost, c->stream));
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  return G2B_OK;
}

int g2b_weights_upload(g2b_ctx *c, const void *host, uint64_t bytes, void **dev) {
  if (!c || !dev || bytes == 0) return fail(c, G2B_EINVAL, "bad weights_upload arguments");
  *dev = nullptr;
  if (int rc = set_device(c)) return rc;
  void *p = nullptr;
  if (hipMalloc(&p, (size_t)bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(c, G2B_ENOMEM, "hipMalloc of %llu weight bytes failed",
                (unsigned long long)bytes);
  }
  if (host) {
    const hipError_t e = hipMemcpy(p, host, (size_t)bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(p);
      return fail(c, G2B_EDEVICE, "weight upload: %s", hipGetErrorString(e));
    }
  }
  *dev = p;
  return G2B_OK;
}

int g2b_weights_free(g2b_ctx *c, void *dev) {
  if (!c) return G2B_EINVAL;
  if (!dev) return G2B_OK;
  if (int rc = set_device(c)) return rc;
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  G2B_HIP(c, hipFree(dev));
  return G2B_OK;
}

int g2b_hbm_info(g2b_ctx *c, uint64_t *free_bytes, uint64_t *total_bytes) {
  if (!c || !free_bytes || !total_bytes) return fail(c, G2B_EINVAL, "bad hbm_info arguments");
  if (int rc = set_device(c)) return rc;
  size_t fr = 0, tot = 0;
  G2B_HIP(c, hipMemGetInfo(&fr, &tot));
  *free_bytes = fr;
  *total_bytes = tot;
  return G2B_OK;
}

int g2b_synth_normal(g2b_ctx *c, float *out, uint64_t n, uint64_t seed) {
  if (!c || (!out && n)) return fail(c, G2B_EINVAL, "bad synth_normal arguments");
  if (int rc = set_device(c)) return rc;
  G2B_HIP(c, launch_synth_normal(out, n, seed, c->stream));
  return G2B_OK;
}

int g2b_synth_fill_kv(g2b_ctx *c, void *kc, void *vc, int32_t ctx_cap, int32_t layer0,
                      int32_t n_layers, int32_t pos0, int32_t n_pos, uint64_t base_seed,
                      int32_t seq, float sel_threshold) {
  if (!c) return G2B_EINVAL;
  if (!kc || !vc) return fail(c, G2B_ENOKV, "KV cache not allocated");
  if (layer0 < 0 || n_layers < 1 || layer0 + n_layers > c->shape.n_layers || n_pos < 0)
    return fail(c, G2B_EINVAL, "bad synth_fill_kv range");
  if (pos0 < 0 || (int64_t)pos0 + n_pos > ctx_cap)
    return fail(c, G2B_EPOS, "rows [%d,%d) outside [0,%d)", pos0, pos0 + n_pos, ctx_cap);
  if (n_pos == 0) return G2B_OK;
  if (int rc = set_device(c)) return rc;
  if (int rc = ensure_rope(c, pos0 + n_pos)) return rc;
  SynthParams sp{};
  sp.sh = c->sh;
  sp.k = (uint8_t *)kc;
  sp.v = (uint8_t *)vc;
  sp.ctx_cap = ctx_cap;
  sp.layer0 = layer0;
  sp.pos0 = pos0;
  sp.n_pos = n_pos;
  sp.base_seed = base_seed;
  sp.seq = seq;
  sp.sel_threshold = sel_threshold;
  sp.rope = c->rope;
  G2B_HIP(c, launch_synth_fill(sp, n_layers, c->stream));
  return G2B_OK;
}

int g2b_synth_copy(g2b_ctx *c, void *dst, const void *src, uint64_t nbytes) {
  if (!c || !dst || !src || (nbytes & 15) || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15))
    return fail(c, G2B_EINVAL, "copy needs 16-byte multiples and alignment");
  if (int rc = set_device(c)) return rc;
  G2B_HIP(c, launch_copy16(dst, src, nbytes / 16, c->stream));
  return G2B_OK;
}

int g2b_ctx_tune(g2b_ctx *c, int32_t split_len, int32_t chunk, int32_t stage, int32_t piece) {
  if (!c || split_len < 0 || (chunk != 0 && chunk != 16 && chunk != 32) || stage < -1 ||
      stage > 2 || piece < -1)
    return G2B_EINVAL;
  c->split_override = split_len;
  c->tune_chunk = chunk;
  c->tune_stage = stage;
  c->tune_piece = piece;
  return G2B_OK;
}

int g2b_ctx_tune_kernel(g2b_ctx *c, int32_t kernel) {
  if (!c || kernel < 0 || kernel > 3) return G2B_EINVAL;
  c->tune_kernel = kernel;
  return G2B_OK;
}

int g2b_ctx_last_schedule(const g2b_ctx *c, int32_t *out) {
  if (!c || !out) return G2B_EINVAL;
  for (int i = 0; i < G2B_SCHED_FIELDS; i++) out[i] = c->sched[i];
  return G2B_OK;
}

int g2b_ctx_profile(g2b_ctx *c, int32_t enable) {
  if (!c) return G2B_EINVAL;
  c->prof = enable != 0;
  c->prof_used = 0;
  return G2B_OK;
}

int g2b_ctx_profile_read(g2b_ctx *c, double *decode_ms, int64_t *launches) {
  if (!c || !decode_ms || !launches) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  double total = 0.0;
  for (size_t i = 0; i + 1 < c->prof_used; i += 2) {
    G2B_HIP(c, hipEventSynchronize(c->prof_ev[i + 1]));
    float ms = 0.f;
    G2B_HIP(c, hipEventElapsedTime(&ms, c->prof_ev[i], c->prof_ev[i + 1]));
    total += ms;
  }
  *decode_ms = total;
  *launches = (int64_t)(c->prof_used / 2);
  c->prof_used = 0;
  return G2B_OK;
}

#ifdef G2B_STAMPS
// The phase-stamp build's own entry points (libg2b_attn_stamps.so; not part
// of the ABI of include/, no counterpart in the reference): room for the
// stamps of `launches` decode calls, each cap workgroups of a k_layer launch
// and as many of its combine, all words zero; g2b_stamps_read synchronises
// the stream, copies out launches * 2 * cap * kStampWords words (call i
// since the previous read in region i) and starts the next calls at region 0.
int g2b_stamps_enable(g2b_ctx *c, int32_t cap, int32_t launches) {
  if (!c || cap < 1 || launches < 1) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  if (c->stamps) G2B_HIP(c, hipFree(c->stamps));
  c->stamps = nullptr;
  c->stamp_cap = c->stamp_launches = c->stamp_next = 0;
  const size_t bytes = (size_t)launches * 2 * cap * kStampWords * sizeof(uint64_t);
  if (hipMalloc((void **)&c->stamps, bytes) != hipSuccess) {
    c->stamps = nullptr;
    (void)hipGetLastError();
    return fail(c, G2B_ENOMEM, "phase stamps");
  }
  G2B_HIP(c, hipMemset(c->stamps, 0, bytes));
  c->stamp_cap = cap;
  c->stamp_launches = launches;
  return G2B_OK;
}

int g2b_stamps_read(g2b_ctx *c, uint64_t *host, int32_t clear) {
  if (!c || !host || !c->stamps) return G2B_EINVAL;
  if (int rc = set_device(c)) return rc;
  const size_t bytes =
      (size_t)c->stamp_launches * 2 * c->stamp_cap * kStampWords * sizeof(uint64_t);
  G2B_HIP(c, hipStreamSynchronize(c->stream));
  c->stamp_next = 0;
  G2B_HIP(c, hipMemcpy(host, c->stamps, bytes, hipMemcpyDeviceToHost));
  if (clear) G2B_HIP(c, hipMemset(c->stamps, 0, bytes));
  return G2B_OK;
}
#endif

}  // extern "C"
