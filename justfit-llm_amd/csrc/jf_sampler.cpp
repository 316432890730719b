// Host side of the C ABI (include/jf_sampler.h): argument checks with the
// reference's messages, per-row kernel parameters, the device penalty table,
// staged uploads and the launches of jf_kernels.hip.
#include "jf_sampler.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <utility>
#include <vector>

#include "jf_host.h"
#include "jf_kernels.h"

namespace {

int fail(int code, const std::string &message) { return jf::set_error(code, message); }

int hip_fail(hipError_t e, const char *what) {
  return fail(JF_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define JF_HIP(call, what)                       \
  do {                                           \
    const hipError_t e_ = (call);                \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// Pinned host slots for asynchronous parameter uploads. A slot is reused
// only after the copy that last read it has completed.
class StagingRing {
 public:
  ~StagingRing() { release(); }

  int upload(void *device_dst, const void *src, size_t bytes,
             hipStream_t stream) {
    if (!bytes) return JF_OK;
    Slot &slot = slots_[next_];
    next_ = (next_ + 1) % kSlots;
    if (slot.pending) {
      JF_HIP(hipEventSynchronize(slot.event), "staging wait");
      slot.pending = false;
    }
    if (slot.capacity < bytes) {
      if (slot.host) JF_HIP(hipHostFree(slot.host), "staging free");
      slot.host = nullptr;
      slot.capacity = 0;
      size_t cap = 4096;
      while (cap < bytes) cap <<= 1;
      JF_HIP(hipHostMalloc(&slot.host, cap, hipHostMallocDefault),
             "staging alloc");
      slot.capacity = cap;
    }
    if (!slot.event)
      JF_HIP(hipEventCreateWithFlags(&slot.event, hipEventDisableTiming),
             "staging event");
    std::memcpy(slot.host, src, bytes);
    JF_HIP(hipMemcpyAsync(device_dst, slot.host, bytes, hipMemcpyHostToDevice,
                          stream),
           "parameter upload");
    JF_HIP(hipEventRecord(slot.event, stream), "staging record");
    slot.pending = true;
    return JF_OK;
  }

  void release() {
    for (Slot &slot : slots_) {
      if (slot.pending && slot.event) (void)hipEventSynchronize(slot.event);
      if (slot.event) (void)hipEventDestroy(slot.event);
      if (slot.host) (void)hipHostFree(slot.host);
      slot = Slot{};
    }
  }

 private:
  static constexpr int kSlots = 8;
  struct Slot {
    void *host = nullptr;
    size_t capacity = 0;
    hipEvent_t event = nullptr;
    bool pending = false;
  };
  Slot slots_[kSlots];
  int next_ = 0;
};

// Host-mapped buffers a kernel reads directly (coherent pinned memory, no
// copy): a slot is refilled only after the event recorded behind the last
// launch that read it has completed.
class MappedRing {
 public:
  ~MappedRing() { release(); }

  // A slot of at least `bytes` for the caller to fill at *host; *device
  // receives the address the kernel reads. Waits for the slot's last reader
  // and allocates before returning, so a failure leaves nothing changed.
  // record() must follow the launch.
  int acquire(size_t bytes, void **host, const void **device) {
    Slot &slot = slots_[next_];
    if (slot.pending) {
      JF_HIP(hipEventSynchronize(slot.event), "mapped batch wait");
      slot.pending = false;
    }
    if (slot.capacity < bytes) {
      if (slot.host) JF_HIP(hipHostFree(slot.host), "mapped batch free");
      slot.host = nullptr;
      slot.capacity = 0;
      size_t cap = 4096;
      while (cap < bytes) cap <<= 1;
      JF_HIP(hipHostMalloc(&slot.host, cap, hipHostMallocCoherent | hipHostMallocMapped),
             "mapped batch alloc");
      slot.capacity = cap;
      JF_HIP(hipHostGetDevicePointer(&slot.device, slot.host, 0), "mapped batch address");
    }
    if (!slot.event)
      JF_HIP(hipEventCreateWithFlags(&slot.event, hipEventDisableTiming), "mapped batch event");
    *host = slot.host;
    *device = slot.device;
    return JF_OK;
  }

  int record(hipStream_t stream) {
    Slot &slot = slots_[next_];
    next_ = (next_ + 1) % kSlots;
    JF_HIP(hipEventRecord(slot.event, stream), "mapped batch record");
    slot.pending = true;
    return JF_OK;
  }

  void release() {
    for (Slot &slot : slots_) {
      if (slot.pending && slot.event) (void)hipEventSynchronize(slot.event);
      if (slot.event) (void)hipEventDestroy(slot.event);
      if (slot.host) (void)hipHostFree(slot.host);
      slot = Slot{};
    }
  }

 private:
  static constexpr int kSlots = 4;
  struct Slot {
    void *host = nullptr;
    void *device = nullptr;
    size_t capacity = 0;
    hipEvent_t event = nullptr;
    bool pending = false;
  };
  Slot slots_[kSlots];
  int next_ = 0;
};

template <class T>
int device_alloc(T **p, size_t count, const char *what) {
  *p = nullptr;
  if (!count) return JF_OK;
  JF_HIP(hipMalloc((void **)p, count * sizeof(T)), what);
  return JF_OK;
}

constexpr uint32_t kMaxRows = 1u << 22;

bool penalties_active(const jf_policy &p) {
  return p.repetition != 1.0f || p.presence != 0.0f || p.frequency != 0.0f;
}

uint32_t effective_top_k(const jf_policy &p, uint32_t vocabulary) {
  return p.top_k && p.top_k < vocabulary ? p.top_k : vocabulary;
}

}  // namespace

// Fixed penalty slots a chunk at most (two per thread of the fast kernel).
constexpr uint32_t kMaxSlots = 2 * jf::kThreads;

struct jf_penalty_table {
  uint32_t vocabulary = 0;
  uint32_t rows = 0;
  uint32_t max_entries = 0;
  uint32_t buckets = 0;
  int device = 0;
  uint2 *entries = nullptr;    // [rows][max_entries] {token, word}
  uint32_t *offsets = nullptr; // [rows][buckets + 1]
  // The fast kernel's fixed slots: [rows][chunks][slot_count], 8192-token
  // chunks; host.fits(row) when every chunk of the row fits its slots and
  // every count fits the slot's 18 bits (otherwise select_kernel takes the
  // row). The array holds room for 512 slots a chunk; a table laid out 256
  // to a chunk widens to 512 when a row needs more (a history clustered in
  // one chunk's ids) and 512 suffice.
  uint32_t chunks = 0;
  uint32_t slot_count = 0;
  uint32_t *slots = nullptr;
  jf::PenaltyRows host;  // the rows as the device holds them
  // Rows a failed count may have left different on the device than in the
  // host copy: refused by jf_sample and by counts until rebuilt.
  std::vector<uint8_t> stale;
  StagingRing staging;
  MappedRing mapped;  // counts of more than kPenaltyOps tokens a call
};

struct jf_sampler {
  uint32_t vocabulary = 0;
  uint32_t max_rows = 0;
  uint32_t max_chunks = 0;
  int device = 0;
  jf::RowParams *params = nullptr;
  jf::BlockHeader *headers = nullptr;
  uint64_t *cands = nullptr;
  uint32_t *counters = nullptr;
  uint64_t *bests = nullptr;
  jf::RowState *states = nullptr;
  jf::StagePartial *partials = nullptr;
  uint64_t workspace_bytes = 0;
  std::vector<jf::RowParams> last_params;
  std::vector<jf::RowParams> host_params;  // the call's rows, reused across calls
  bool params_valid = false;
  StagingRing staging;
  // Set to 1 by a greedy finisher whose bounded wait gave up (coherent
  // host-mapped memory: the host reads it without a device synchronization).
  uint32_t *status_host = nullptr;
  uint32_t *status_device = nullptr;
  uint32_t epoch = 0;                 // the last call's tag, 1..4095
  uint32_t wait_bound = 1u << 20;     // reads of a packed best before giving up
  // Drafted rows' weights stored by the select pass for their residual pass
  // (lean_rows rows x max_chunks x 8192 words), allocated on first need.
  uint32_t *lean_weights = nullptr;
  uint32_t lean_rows = 0;
};

extern "C" {

// ---- sampler -------------------------------------------------------------

int jf_sampler_destroy(jf_sampler *s) {
  if (!s) return JF_OK;
  s->staging.release();
  (void)hipFree(s->params);
  (void)hipFree(s->headers);
  (void)hipFree(s->cands);
  (void)hipFree(s->counters);
  (void)hipFree(s->bests);
  (void)hipFree(s->states);
  (void)hipFree(s->partials);
  (void)hipFree(s->lean_weights);
  if (s->status_host) (void)hipHostFree(s->status_host);
  delete s;
  return JF_OK;
}

int jf_sampler_create(uint32_t vocabulary, uint32_t max_rows,
                      jf_sampler **out) {
  if (!out) return fail(JF_ERR_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (!vocabulary) return fail(JF_ERR_INVALID_ARGUMENT, "invalid sampling geometry");
  if (!max_rows) return fail(JF_ERR_INVALID_ARGUMENT, "invalid sampling workspace row count");
  // The fast selection launch packs its first row, in units of 256 rows,
  // into 14 bits of one kernel argument.
  if (max_rows > kMaxRows)
    return fail(JF_ERR_INVALID_ARGUMENT, "sampling workspace row count exceeds 4194304");
  const uint32_t max_chunks = (vocabulary + jf::kChunkF32 - 1) / jf::kChunkF32;
  if (max_chunks > 64)
    return fail(JF_ERR_INVALID_ARGUMENT, "vocabulary exceeds 524288 tokens");
  jf_sampler *s = new (std::nothrow) jf_sampler;
  if (!s) return fail(JF_ERR_NO_MEMORY, "sampler allocation failed");
  s->vocabulary = vocabulary;
  s->max_rows = max_rows;
  s->max_chunks = max_chunks;
  int rc = JF_OK;
  const hipError_t ge = hipGetDevice(&s->device);
  if (ge != hipSuccess) rc = hip_fail(ge, "hipGetDevice");
  const uint64_t blocks = (uint64_t)max_rows * max_chunks;
  if (rc == JF_OK) rc = device_alloc(&s->params, max_rows, "row parameters");
  if (rc == JF_OK) rc = device_alloc(&s->headers, blocks, "block headers");
  if (rc == JF_OK) rc = device_alloc(&s->cands, blocks * jf::kBlockCandidates, "candidates");
  if (rc == JF_OK) rc = device_alloc(&s->counters, max_rows, "arrival counters");
  if (rc == JF_OK) rc = device_alloc(&s->bests, blocks, "greedy bests");
  if (rc == JF_OK) rc = device_alloc(&s->states, max_rows, "row states");
  if (rc == JF_OK) rc = device_alloc(&s->partials, blocks, "stage partials");
  if (rc == JF_OK) {
    const hipError_t e =
        hipHostMalloc((void **)&s->status_host, sizeof(uint32_t),
                      hipHostMallocCoherent | hipHostMallocMapped);
    if (e != hipSuccess) {
      s->status_host = nullptr;
      rc = hip_fail(e, "status word");
    } else {
      *s->status_host = 0;
      const hipError_t e2 = hipHostGetDevicePointer((void **)&s->status_device, s->status_host, 0);
      if (e2 != hipSuccess) rc = hip_fail(e2, "status word address");
    }
  }
  if (rc == JF_OK) {
    const hipError_t e1 = hipMemset(s->counters, 0, max_rows * sizeof(uint32_t));
    const hipError_t e2 = hipMemset(s->states, 0, max_rows * sizeof(jf::RowState));
    const hipError_t e4 = hipMemset(s->bests, 0, blocks * sizeof(uint64_t));
    // The fused draw's self-validating summary words start as zero too.
    const hipError_t e5 = hipMemset(s->partials, 0, blocks * sizeof(jf::StagePartial));
    const hipError_t e3 = hipDeviceSynchronize();
    if (e1 != hipSuccess) rc = hip_fail(e1, "counter init");
    else if (e2 != hipSuccess) rc = hip_fail(e2, "state init");
    else if (e4 != hipSuccess) rc = hip_fail(e4, "greedy best init");
    else if (e5 != hipSuccess) rc = hip_fail(e5, "chunk summary init");
    else if (e3 != hipSuccess) rc = hip_fail(e3, "init sync");
  }
  if (rc != JF_OK) {
    jf_sampler_destroy(s);
    return rc;
  }
  s->workspace_bytes =
      max_rows * (sizeof(jf::RowParams) + sizeof(uint32_t) + sizeof(jf::RowState)) +
      blocks * (sizeof(jf::BlockHeader) + jf::kBlockCandidates * sizeof(uint64_t) +
                sizeof(uint64_t) + sizeof(jf::StagePartial));
  *out = s;
  return JF_OK;
}

uint64_t jf_sampler_workspace_bytes(const jf_sampler *s) {
  return s ? s->workspace_bytes +
                 (uint64_t)s->lean_rows * s->max_chunks * jf::kChunkF32 * sizeof(uint32_t)
           : 0;
}

static int check_device(int device) {
  int current = -1;
  JF_HIP(hipGetDevice(&current), "hipGetDevice");
  if (current != device)
    return fail(JF_ERR_INVALID_ARGUMENT,
                "call made on a different device than the object was created on");
  return JF_OK;
}

// ---- penalties -------------------------------------------------------------

int jf_penalty_table_destroy(jf_penalty_table *t) {
  if (!t) return JF_OK;
  t->staging.release();
  t->mapped.release();
  (void)hipFree(t->entries);
  (void)hipFree(t->offsets);
  (void)hipFree(t->slots);
  delete t;
  return JF_OK;
}

int jf_penalty_table_create(uint32_t vocabulary, uint32_t rows,
                            uint32_t max_entries, jf_penalty_table **out) {
  if (!out) return fail(JF_ERR_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (!vocabulary || !rows || !max_entries || max_entries > 0x7fffffffu)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid penalty table geometry");
  jf_penalty_table *t = new (std::nothrow) jf_penalty_table;
  if (!t) return fail(JF_ERR_NO_MEMORY, "penalty table allocation failed");
  t->vocabulary = vocabulary;
  t->rows = rows;
  t->max_entries = max_entries;
  t->buckets = (vocabulary + jf::kPenaltyBucket - 1) / jf::kPenaltyBucket;
  t->chunks = (vocabulary + jf::kChunkF32 - 1) / jf::kChunkF32;
  // Half again the mean entries of a chunk, in whole slots per thread.
  t->slot_count = (uint64_t)max_entries * 3 / 2 <= (uint64_t)t->chunks * jf::kThreads
                      ? (uint32_t)jf::kThreads
                      : 2u * jf::kThreads;
  t->host.init(vocabulary, rows, max_entries, t->slot_count);
  t->stale.assign(rows, 0);
  int rc = JF_OK;
  hipError_t ge = hipGetDevice(&t->device);
  if (ge != hipSuccess) rc = hip_fail(ge, "hipGetDevice");
  if (rc == JF_OK) rc = device_alloc(&t->entries, (size_t)rows * max_entries, "penalty entries");
  if (rc == JF_OK) rc = device_alloc(&t->offsets, (size_t)rows * (t->buckets + 1), "penalty offsets");
  const size_t slot_room = (size_t)rows * t->chunks * kMaxSlots;
  if (rc == JF_OK) rc = device_alloc(&t->slots, slot_room, "penalty slots");
  if (rc == JF_OK) {
    ge = hipMemset(t->offsets, 0, (size_t)rows * (t->buckets + 1) * sizeof(uint32_t));
    if (ge == hipSuccess) ge = hipMemset(t->slots, 0, slot_room * sizeof(uint32_t));
    if (ge == hipSuccess) ge = hipDeviceSynchronize();
    if (ge != hipSuccess) rc = hip_fail(ge, "penalty table init");
  }
  if (rc != JF_OK) {
    jf_penalty_table_destroy(t);
    return rc;
  }
  *out = t;
  return JF_OK;
}

// The row's fixed slots as the host copy lays them out.
static int upload_penalty_slots(jf_penalty_table *t, uint32_t row, void *stream) {
  const size_t per_row = (size_t)t->chunks * t->slot_count;
  std::vector<uint32_t> sl(per_row);
  t->host.slots(row, sl.data());
  return t->staging.upload(t->slots + (size_t)row * per_row, sl.data(),
                           per_row * sizeof(uint32_t), (hipStream_t)stream);
}

// Widens a table of 256 slots a chunk to 512 once some row needs more than
// 256 and fits 512: every row that fits then is laid out again (after the
// updates already on `stream`).
static int widen_slots(jf_penalty_table *t, void *stream) {
  if (t->slot_count >= kMaxSlots) return JF_OK;
  bool wider = false;
  for (uint32_t r = 0; r < t->rows && !wider; ++r)
    wider = !t->host.fits(r) && t->host.size(r) > 0 && t->host.fits_at(r, kMaxSlots);
  if (!wider) return JF_OK;
  t->slot_count = kMaxSlots;
  t->host.set_slot_count(kMaxSlots);
  for (uint32_t r = 0; r < t->rows; ++r) {
    if (!t->host.fits(r)) continue;
    const int rc = upload_penalty_slots(t, r, stream);
    if (rc != JF_OK) {
      // This row and the later ones keep the narrower layout on the device.
      for (uint32_t q = r; q < t->rows; ++q) t->stale[q] = 1;
      return rc;
    }
  }
  return JF_OK;
}

// The whole row as the host copy holds it: entries, bucket offsets, and
// the fixed slots when the row fits them.
static int upload_penalty_row(jf_penalty_table *t, uint32_t row, void *stream) {
  const uint32_t n = t->host.size(row);
  std::vector<uint8_t> blob(n * sizeof(uint2) + (t->buckets + 1) * sizeof(uint32_t));
  uint32_t *off = (uint32_t *)(blob.data() + n * sizeof(uint2));
  t->host.entries(row, (jf::PenaltyEntry *)blob.data());
  t->host.offsets(row, off);
  const hipStream_t st = (hipStream_t)stream;
  int rc = t->staging.upload(t->entries + (size_t)row * t->max_entries, blob.data(),
                             n * sizeof(uint2), st);
  if (rc != JF_OK) return rc;
  rc = t->staging.upload(t->offsets + (size_t)row * (t->buckets + 1), off,
                         (t->buckets + 1) * sizeof(uint32_t), st);
  if (rc != JF_OK || !t->host.fits(row)) return rc;
  return upload_penalty_slots(t, row, stream);
}

int jf_penalty_table_rebuild(jf_penalty_table *t, uint32_t row,
                             const uint32_t *history, uint64_t history_len,
                             uint64_t generated, int has_pending,
                             uint32_t pending, int mark_prompt, void *stream) {
  if (!t) return fail(JF_ERR_INVALID_ARGUMENT, "penalty table is null");
  if (row >= t->rows)
    return fail(JF_ERR_INVALID_ARGUMENT, "penalized lane has no penalty table row");
  int rc = check_device(t->device);
  if (rc != JF_OK) return rc;
  std::vector<uint32_t> words(t->vocabulary);
  rc = jf_penalty_words_rebuild(words.data(), t->vocabulary, history, history_len,
                                generated, has_pending, pending, mark_prompt);
  if (rc != JF_OK) return rc;
  rc = t->host.rebuild(row, words.data());
  if (rc != JF_OK) return rc;
  rc = upload_penalty_row(t, row, stream);
  if (rc != JF_OK) {
    t->stale[row] = 1;
    return rc;
  }
  t->stale[row] = 0;
  return widen_slots(t, stream);
}

// The update of one (row, token) pair as penalty_count_kernel reads it.
static int count_op(jf_penalty_table *t, uint32_t row, uint32_t token,
                    jf::PackedPenaltyOp *p) {
  jf::PenaltyOp op;
  const int rc = t->host.count(row, token, &op);
  if (rc != JF_OK) return rc;
  p->token = op.token;
  p->word = op.word;
  p->index = op.index | (op.insert ? 0x80000000u : 0u);
  p->entries = op.entries;
  p->slot_value = op.slot_value;
  p->slot = op.slot == jf::kNoSlot ? 0xffffu : (op.slot | op.slot_used << 16);
  return JF_OK;
}

// More tokens than one kernel-argument batch holds: every update in one
// launch that reads them from host-mapped memory (ops, group rows, group
// starts), so a step's commits of many lanes cost one kernel.
static int count_mapped(jf_penalty_table *t, const jf::PenaltyTableView &view,
                        const uint32_t *rows, uint32_t one_row, const uint32_t *selected,
                        const std::vector<uint64_t> &order, void *stream) {
  const uint64_t n = order.size();
  std::vector<uint32_t> group_row, group_start;
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t row = rows ? rows[order[i]] : one_row;
    if (group_row.empty() || group_row.back() != row) {
      group_row.push_back(row);
      group_start.push_back((uint32_t)i);
    }
  }
  group_start.push_back((uint32_t)n);
  const size_t ob = n * sizeof(jf::PackedPenaltyOp), rb = group_row.size() * sizeof(uint32_t),
               sb = group_start.size() * sizeof(uint32_t);
  // The buffer first (its wait or allocation may fail): the host copy
  // changes only once the updates have somewhere to go.
  void *host = nullptr;
  const void *dev = nullptr;
  int rc = t->mapped.acquire(ob + rb + sb, &host, &dev);
  if (rc != JF_OK) return rc;
  uint8_t *h = (uint8_t *)host;
  jf::PackedPenaltyOp *ops = (jf::PackedPenaltyOp *)h;
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t k = order[i];
    rc = count_op(t, rows ? rows[k] : one_row, selected[k], &ops[i]);
    if (rc != JF_OK) return rc;  // excluded by the caller's checks
  }
  std::memcpy(h + ob, group_row.data(), rb);
  std::memcpy(h + ob + rb, group_start.data(), sb);
  const uint8_t *d = (const uint8_t *)dev;
  const int e = jf::launch_penalty_count_mapped(
      view, (const jf::PackedPenaltyOp *)d, (const uint32_t *)(d + ob),
      (const uint32_t *)(d + ob + rb), (uint32_t)group_row.size(), stream);
  if (e != hipSuccess) return hip_fail((hipError_t)e, "penalty count launch");
  rc = t->mapped.record((hipStream_t)stream);
  return rc == JF_OK ? widen_slots(t, stream) : rc;
}

// countPenaltyTokens (Sampling.cpp:75-80) of n (row, token) pairs, applied
// in order. Everything is checked before any row changes: rows, tokens, and
// that each row's new distinct tokens fit its max_entries. The host copy
// then describes each token's update, and penalty_count_kernel applies them
// on `stream` in one launch: as kernel arguments (up to kPenaltyOps tokens,
// no copy and no wait on earlier work) or from host-mapped memory.
static int count_pairs_checked(jf_penalty_table *t, const uint32_t *rows, uint32_t one_row,
                               const uint32_t *selected, uint64_t n, void *stream);

static int count_pairs(jf_penalty_table *t, const uint32_t *rows, uint32_t one_row,
                       const uint32_t *selected, uint64_t n, void *stream) {
  if (!selected && n) return fail(JF_ERR_INVALID_ARGUMENT, "null buffer");
  int rc = check_device(t->device);
  if (rc != JF_OK) return rc;
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t row = rows ? rows[i] : one_row;
    if (row >= t->rows)
      return fail(JF_ERR_INVALID_ARGUMENT, "penalized lane has no penalty table row");
    if (selected[i] >= t->vocabulary)
      return fail(JF_ERR_INVALID_ARGUMENT, "penalty token is outside the vocabulary");
    if (t->stale[row])
      return fail(JF_ERR_LOGIC, "penalty table row is out of date after a failed update; "
                                "rebuild it");
    t->host.prefetch(row, selected[i]);
  }
  rc = count_pairs_checked(t, rows, one_row, selected, n, stream);
  if (rc == JF_ERR_DEVICE) {
    // A launch or an upload failed after the host copy took some of the
    // updates: the device rows may differ from it.
    for (uint64_t i = 0; i < n; ++i) t->stale[rows ? rows[i] : one_row] = 1;
  }
  return rc;
}

// count_pairs after its argument checks.
static int count_pairs_checked(jf_penalty_table *t, const uint32_t *rows, uint32_t one_row,
                               const uint32_t *selected, uint64_t n, void *stream) {
  int rc = JF_OK;
  // Updates grouped by row, call order kept inside each row.
  std::vector<uint64_t> order(n);
  for (uint64_t i = 0; i < n; ++i) order[i] = i;
  if (rows)
    std::stable_sort(order.begin(), order.end(),
                     [&](uint64_t x, uint64_t y) { return rows[x] < rows[y]; });
  // Each row's new distinct tokens must fit its max_entries. A row whose
  // size plus its token count fits cannot overflow; only the others look
  // their tokens up.
  std::vector<uint32_t> fresh;
  for (uint64_t i = 0; i < n;) {
    const uint32_t row = rows ? rows[order[i]] : one_row;
    uint64_t j = i;
    while (j < n && (rows ? rows[order[j]] : one_row) == row) ++j;
    if (t->host.size(row) + (j - i) > t->max_entries) {
      fresh.clear();
      for (uint64_t k = i; k < j; ++k)
        if (!t->host.holds(row, selected[order[k]])) fresh.push_back(selected[order[k]]);
      std::sort(fresh.begin(), fresh.end());
      const size_t distinct = std::unique(fresh.begin(), fresh.end()) - fresh.begin();
      if (t->host.size(row) + distinct > t->max_entries)
        return fail(JF_ERR_INVALID_ARGUMENT, "penalty history exceeds the table row");
    }
    i = j;
  }
  const jf::PenaltyTableView view{(jf::PenaltyEntry *)t->entries, t->offsets, t->slots,
                                  t->max_entries, t->buckets, t->chunks, t->slot_count};
  jf::PenaltyOpBatch b;
  uint32_t ops = 0, groups = 0;
  auto flush = [&]() -> int {
    if (!ops) return JF_OK;
    b.group_start[groups] = ops;
    const int e = jf::launch_penalty_count(view, b, groups, stream);
    ops = groups = 0;
    return e == hipSuccess ? JF_OK : hip_fail((hipError_t)e, "penalty count launch");
  };
  if (n > jf::kPenaltyOps) return count_mapped(t, view, rows, one_row, selected, order, stream);
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t k = order[i];
    const uint32_t row = rows ? rows[k] : one_row;
    if (ops == jf::kPenaltyOps) {
      rc = flush();
      if (rc != JF_OK) return rc;
    }
    if (!ops || b.group_row[groups - 1] != row) {
      b.group_row[groups] = row;
      b.group_start[groups++] = ops;
    }
    rc = count_op(t, row, selected[k], &b.op[ops++]);
    if (rc != JF_OK) return rc;  // excluded by the checks above
  }
  rc = flush();
  return rc == JF_OK ? widen_slots(t, stream) : rc;
}

int jf_penalty_table_count(jf_penalty_table *t, uint32_t row,
                           const uint32_t *selected, uint64_t count,
                           void *stream) {
  if (!t) return fail(JF_ERR_INVALID_ARGUMENT, "penalty table is null");
  if (row >= t->rows)
    return fail(JF_ERR_INVALID_ARGUMENT, "penalized lane has no penalty table row");
  return count_pairs(t, nullptr, row, selected, count, stream);
}

int jf_penalty_table_count_rows(jf_penalty_table *t, const uint32_t *rows,
                                const uint32_t *selected, uint64_t count, void *stream) {
  if (!t) return fail(JF_ERR_INVALID_ARGUMENT, "penalty table is null");
  if (!rows && count) return fail(JF_ERR_INVALID_ARGUMENT, "null buffer");
  return count_pairs(t, rows, 0, selected, count, stream);
}

// ---- selection ---------------------------------------------------------

}  // extern "C"

namespace jf {

int sample_core(uint32_t V, const SampleScratch &sc, const jf_sample_args *a,
                RowParams *params, ParamUpload upload, void *upload_ctx,
                void *stream, const AcceptTreeLaunch *accept, bool *accepted) {
  if (accepted) *accepted = false;
  int rc = JF_OK;
  const uint32_t rows = a->rows;
  if (!rows || rows > sc.max_rows)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid sampling batch width");
  if ((V + kChunkF32 - 1) / kChunkF32 > sc.max_chunks)
    return fail(JF_ERR_INVALID_ARGUMENT, "vocabulary exceeds the sampling scratch");
  if (a->dtype != JF_DTYPE_F32 && a->dtype != JF_DTYPE_BF16)
    return fail(JF_ERR_INVALID_ARGUMENT, "unsupported logits dtype");
  if (!a->logits || !a->policies || !a->out_tokens)
    return fail(JF_ERR_INVALID_ARGUMENT, "null logits, policies or output tokens");
  const uint64_t esize = a->dtype == JF_DTYPE_F32 ? 4 : 2;
  if (rows > 1 && a->logits_stride < V)
    return fail(JF_ERR_INVALID_ARGUMENT, "logits row stride is below the vocabulary");
  if ((uintptr_t)a->logits % esize)
    return fail(JF_ERR_INVALID_ARGUMENT, "logits are not aligned to their element size");
  const bool aligned =
      (uintptr_t)a->logits % 16 == 0 && (rows == 1 || (a->logits_stride * esize) % 16 == 0);
  const bool kept = a->out_kept_ids || a->out_kept_probs || a->out_kept_counts;
  if (kept && (!a->out_kept_ids || !a->out_kept_probs || !a->out_kept_counts ||
               !a->kept_capacity))
    return fail(JF_ERR_INVALID_ARGUMENT,
                "kept outputs need ids, probabilities, counts and a capacity");
  const uint32_t W = (V + 31) / 32;
  bool any_constrained = false, any_sampled = false, staged = false, any_drafted = false;
  const bool row_indexed = a->draft_token_index || a->draft_cand_index;
  bool need_count1 = false, need_topk = false, need_topp = false;
  for (uint32_t r = 0; r < rows; ++r) {
    const jf_policy &p = a->policies[r];
    rc = jf_policy_validate(&p);
    if (rc != JF_OK) return rc;
    jf::RowParams rp{};
    const bool sampled = p.temperature > 0.0f;
    if (sampled) {
      rp.flags |= jf::kRowSampled;
      rp.top_k = effective_top_k(p, V);
      rp.inv_t = 1.0f / p.temperature;
      rp.top_p = p.top_p;
      if (rp.top_k < V) rp.flags |= jf::kRowTopK;
      if (p.top_p < 1.0f) rp.flags |= jf::kRowTopP;
      if (p.min_p > 0.0f) {
        rp.flags |= jf::kRowMinP;
        rp.minp_offset = p.temperature * std::log(p.min_p);
      }
      any_sampled = true;
      if (rp.top_k > (uint32_t)jf::kBlockCandidates) {
        staged = true;
        need_count1 |= (rp.flags & (jf::kRowMinP | jf::kRowTopK)) != 0;
        need_topk |= (rp.flags & jf::kRowTopK) != 0;
        need_topp |= (rp.flags & jf::kRowTopP) != 0;
      }
    }
    if (p.flags & JF_POLICY_CONSTRAINED) {
      rp.flags |= jf::kRowConstrained;
      any_constrained = true;
    }
    if (p.flags & JF_POLICY_EXCLUDE_STOP) rp.flags |= jf::kRowExcludeStop;
    rp.penalty_row = JF_NO_TOKEN;
    rp.mask_row = a->mask_rows ? a->mask_rows[r] : r;
    rp.draft_index = a->draft_token_index ? a->draft_token_index[r]
                     : (a->draft_tokens && r < a->drafted_rows) ? r
                                                                : JF_NO_TOKEN;
    rp.cand_index = a->draft_cand_index ? a->draft_cand_index[r] : r;
    const uint64_t extra_offset =
        a->extra_offsets ? a->extra_offsets[r] : (uint64_t)r * a->extra_stride;
    if (extra_offset > 0xffffffffull)
      return fail(JF_ERR_INVALID_ARGUMENT, "extra token offset exceeds 32 bits");
    rp.extra_offset = (uint32_t)extra_offset;
    if (rp.draft_index != JF_NO_TOKEN) any_drafted = true;
    const uint32_t extra = a->extra_counts ? a->extra_counts[r] : 0u;
    if (extra > (uint32_t)jf::kMaxExtra)
      return fail(JF_ERR_INVALID_ARGUMENT, "more than 16 extra penalty tokens in a row");
    if (extra && !a->extra_tokens)
      return fail(JF_ERR_INVALID_ARGUMENT, "extra penalty tokens are null");
    if (penalties_active(p)) {
      if (!a->penalties || !a->penalty_rows || a->penalty_rows[r] >= a->penalties->rows)
        return fail(JF_ERR_INVALID_ARGUMENT, "penalized lane has no penalty table row");
      if (a->penalties->vocabulary != V)
        return fail(JF_ERR_INVALID_ARGUMENT, "penalty table vocabulary differs");
      if (a->penalties->stale[a->penalty_rows[r]])
        return fail(JF_ERR_LOGIC, "penalty table row is out of date after a failed update; "
                                  "rebuild it");
      rp.flags |= jf::kRowPenalized;
      rp.penalty_row = a->penalty_rows[r];
      rp.extra_count = extra;
      rp.repetition = p.repetition;
      rp.repetition_inverse = std::min(1.0f / p.repetition, FLT_MAX);
      rp.presence = p.presence;
      rp.frequency = p.frequency;
    }
    params[r] = rp;
  }
  if (any_constrained && (!a->masks || (rows > 1 && a->mask_stride < W)))
    return fail(JF_ERR_INVALID_ARGUMENT, "constraint mask buffer is missing or short");
  if (any_sampled && !a->uniforms)
    return fail(JF_ERR_INVALID_ARGUMENT, "sampling uniforms are null");
  if (any_drafted && !a->draft_tokens)
    return fail(JF_ERR_INVALID_ARGUMENT, "drafted rows need draft tokens");
  if (any_drafted && !a->draft_q && (!a->draft_cand_ids || !a->draft_cand_probs))
    return fail(JF_ERR_INVALID_ARGUMENT, "drafted rows need draft probabilities");

  // The rows the fast selection kernel takes: in a launch of 16-byte-aligned
  // rows (and a vocabulary of at least one vector), each row whose penalty
  // row fits its fixed slots and whose extra verify tokens (if any) start
  // below 2^27 (their offset travels in 27 bits of a kernel argument). When
  // only some rows qualify the launch is split: the fast kernel selects
  // those, and select_kernel the others (it skips rows marked fast_row).
  const uint64_t stride_el = rows > 1 ? a->logits_stride : V;
  const bool launch_fast = aligned && V >= 8 && stride_el <= 0xffffffffull &&
                           !(a->mask_rows && any_constrained);
  uint32_t n_fast = 0;
  for (uint32_t r = 0; r < rows; ++r) {
    jf::RowParams &rp = params[r];
    const bool ok = launch_fast && (!rp.extra_count || rp.extra_offset <= jf::kExtraOffsetMask) &&
                    !((rp.flags & jf::kRowPenalized) &&
                      (!a->penalties->host.fits(rp.penalty_row) || rp.penalty_row > 0xffffffu));
    rp.fast_row = ok ? 1u : 0u;
    n_fast += ok ? 1u : 0u;
  }
  const bool fast = n_fast == rows, split = n_fast && !fast;
  if (!split)
    for (uint32_t r = 0; r < rows; ++r) params[r].fast_row = 0;
  // Drafted rows with no cut, penalty, mask or extra tokens: residual_kernel
  // takes their residual pass (kRowLean; no other kernel reads the flag but
  // uncut_kernel).
  uint32_t n_lean = 0;
  for (uint32_t r = 0; r < rows; ++r) {
    jf::RowParams &rp = params[r];
    const bool lean =
        (rp.flags & jf::kRowSampled) && rp.draft_index != JF_NO_TOKEN && !rp.extra_count &&
        !(rp.flags & (jf::kRowMinP | jf::kRowTopK | jf::kRowTopP | jf::kRowPenalized |
                      jf::kRowConstrained));
    rp.flags = lean ? rp.flags | jf::kRowLean : rp.flags & ~jf::kRowLean;
    n_lean += lean ? 1u : 0u;
  }

  rc = upload(upload_ctx, params, rows, sc.params, stream);
  if (rc != JF_OK) return rc;

  jf::SampleLaunch L{};
  L.logits = a->logits;
  L.stride = rows > 1 ? a->logits_stride : V;
  L.masks = a->masks;
  L.mask_stride = a->mask_stride;
  L.params = sc.params;
  L.vocabulary = V;
  L.chunks = (V + (a->dtype == JF_DTYPE_F32 ? jf::kChunkF32 : jf::kChunkBF16) - 1) /
             (a->dtype == JF_DTYPE_F32 ? jf::kChunkF32 : jf::kChunkBF16);
  L.rows = rows;
  L.stop0 = a->stop_token_0;
  L.stop1 = a->stop_token_1;
  L.aligned = aligned ? 1u : 0u;
  if (a->penalties) {
    L.pen_entries = a->penalties->entries;
    L.pen_offsets = a->penalties->offsets;
    L.pen_max_entries = a->penalties->max_entries;
    L.pen_buckets = a->penalties->buckets;
  }
  L.extra = a->extra_tokens;
  L.extra_stride = a->extra_stride;
  L.uniforms = a->uniforms;
  L.uniform_index = a->uniform_index;
  L.uniform_offset = a->uniform_offset;
  L.uniform_stride = a->uniform_stride;
  L.draft_tokens = a->draft_tokens;
  // drafted_rows: nonzero when any row is drafted; the merges' early loads
  // use it as the linear prefix unless the rows are indexed.
  L.drafted_rows = !any_drafted ? 0u : row_indexed ? rows : a->drafted_rows;
  L.row_indexed = row_indexed ? 1u : 0u;
  L.cand_ids = a->draft_cand_ids;
  L.cand_probs = a->draft_cand_probs;
  L.dense_q = a->draft_q;
  L.q_stride = a->draft_q_stride;
  L.headers = sc.headers;
  L.cands = sc.cands;
  L.counters = sc.counters;
  L.bests = sc.bests;
  L.states = sc.states;
  L.partials = sc.partials;
  L.out_tokens = a->out_tokens;
  L.out_draft = a->out_draft_probs;
  L.out_kept_counts = a->out_kept_counts;
  L.out_kept_ids = a->out_kept_ids;
  L.out_kept_probs = a->out_kept_probs;
  L.kept_cap = a->kept_capacity;
  L.q_aligned = a->draft_q && (uintptr_t)a->draft_q % 16 == 0 &&
                        (a->draft_q_stride * sizeof(float)) % 16 == 0
                    ? 1u
                    : 0u;
  L.epoch = sc.epoch;
  L.wait_bound = sc.wait_bound;
  L.status = sc.status;
  // Drafted rows with no cut in an all-fast fp32 launch with no extra
  // tokens: the select pass stores their weights and the residual pass
  // reads them.
  bool any_extra = false;
  for (uint32_t r = 0; r < rows; ++r) any_extra |= params[r].extra_count != 0;
  if (n_lean && fast && !any_extra && a->dtype == JF_DTYPE_F32 && sc.lean_weights) {
    L.lean_weights = sc.lean_weights(upload_ctx, rows);
    L.lean_stride = (uint64_t)L.chunks * jf::kChunkF32;
  }

  if ((a->select_start_event == nullptr) != (a->select_done_event == nullptr))
    return fail(JF_ERR_INVALID_ARGUMENT, "select events come in pairs");
  int e = hipSuccess;
  // A launch of greedy rows only is finished inside the fast selection.
  const bool fused = fast && !any_sampled;
  // Sampled rows that keep every admitted token (no min-p, top-k or top-p
  // cut): the selection writes their chunk masses and uncut_kernel draws
  // them; the merge and the stages finish the other rows and skip these, so
  // only the cut rows decide the merge and the stages.
  constexpr uint32_t kCuts = jf::kRowMinP | jf::kRowTopK | jf::kRowTopP;
  // uncut_drafted: drafted uncut rows whose residual pass stays in
  // uncut_kernel (not kRowLean).
  bool any_uncut = false, any_cut = false, any_greedy = false, uncut_drafted = false;
  staged = need_count1 = need_topk = need_topp = false;
  for (uint32_t r = 0; r < rows; ++r) {
    const jf::RowParams &rp = params[r];
    if (!(rp.flags & jf::kRowSampled)) {
      any_greedy = true;
    } else if (!(rp.flags & kCuts)) {
      any_uncut = true;
      if (rp.draft_index != JF_NO_TOKEN && !(rp.flags & jf::kRowLean)) uncut_drafted = true;
    } else {
      any_cut = true;
      if (rp.top_k > (uint32_t)jf::kBlockCandidates) {
        staged = true;
        need_count1 |= (rp.flags & (jf::kRowMinP | jf::kRowTopK)) != 0;
        need_topk |= (rp.flags & jf::kRowTopK) != 0;
        need_topp |= (rp.flags & jf::kRowTopP) != 0;
      }
    }
  }
  // A fast launch of rows that all keep every admitted token, with no draft,
  // penalty or extra token and no kept outputs: each row's last chunk block
  // draws it, so no uncut_kernel launch follows.
  bool fuse_uncut = fast && any_uncut && !any_cut && !any_greedy && !any_drafted && !kept;
  for (uint32_t r = 0; fuse_uncut && r < rows; ++r)
    fuse_uncut = !(params[r].flags & jf::kRowPenalized) && !params[r].extra_count;
  // The merge finishes the cut rows, and the greedy rows unless the launch
  // is all greedy and fast (fused) or has uncut rows and no cut ones (then
  // uncut_kernel takes them).
  const bool need_merge = !fused && (any_cut || (any_greedy && !any_uncut));
  L.finish_greedy = any_greedy && !need_merge && !fused ? 1u : 0u;
  if (!fast) {
    e = jf::launch_select(L, a->dtype, stream, a->select_start_event,
                          split ? nullptr : a->select_done_event);
  }
  if (e == hipSuccess && (fast || split)) {
    jf::FastLaunch F{};
    thread_local jf::FastRows s_rows;  // copied into the launch's arguments
    F.a = L;
    F.fuse_greedy = fused ? 1u : 0u;
    F.mapped = split ? 1u : 0u;
    if (a->penalties) {
      F.pen_slots = a->penalties->slots;
      F.slot_count = a->penalties->slot_count;
    }
    std::vector<uint32_t> fast_rows;
    if (split) {
      fast_rows.reserve(n_fast);
      for (uint32_t r = 0; r < rows; ++r)
        if (params[r].fast_row) fast_rows.push_back(r);
    }
    auto row_at = [&](uint32_t i) { return split ? fast_rows[i] : i; };
    // A uniform launch: every row has the same policy, and penalized rows
    // read their own table row; the kernel then takes the policy from its
    // preloaded arguments instead of a memory read per block.
    bool uniform = true;
    const jf::RowParams &p0 = params[row_at(0)];
    for (uint32_t i = 0; uniform && i < n_fast; ++i) {
      const uint32_t r = row_at(i);
      const jf::RowParams &p = params[r];
      uniform = ((p.flags ^ p0.flags) & ~jf::kRowLean) == 0 && p.top_k == p0.top_k &&
                p.minp_offset == p0.minp_offset && p.repetition == p0.repetition &&
                p.repetition_inverse == p0.repetition_inverse &&
                p.presence == p0.presence && p.frequency == p0.frequency &&
                (!(p.flags & jf::kRowPenalized) || p.penalty_row == r);
    }
    for (uint32_t i0 = 0; i0 < n_fast && e == hipSuccess; i0 += jf::kKernargRows) {
      const uint32_t n = std::min<uint32_t>(n_fast - i0, jf::kKernargRows);
      F.row_base = split ? 0u : i0;
      bool extras = false;
      std::memset(F.lean_bits, 0, sizeof(F.lean_bits));
      for (uint32_t i = 0; i < n; ++i) {
        const jf::RowParams &rp = params[row_at(i0 + i)];
        extras |= rp.extra_count != 0;
        if (rp.flags & jf::kRowLean) F.lean_bits[i >> 5] |= 1u << (i & 31);
      }
      // Per-row facts only where the kernel reads them (a launch that is not
      // uniform, mapped or with extra tokens).
      const bool rows_arg = !uniform || split || extras;
      if (rows_arg) {
        for (uint32_t i = 0; i < n; ++i) {
          const uint32_t r = row_at(i0 + i);
          const jf::RowParams &rp = params[r];
          const uint32_t prow = (rp.flags & jf::kRowPenalized) ? rp.penalty_row : 0u;
          s_rows.row_info[i] = (rp.flags & 0xffu) | (prow << 8);
          s_rows.row_of[i] = r;
          s_rows.row_extra[i] = rp.extra_count ? rp.extra_offset | rp.extra_count << 27 : 0u;
        }
      }
      const bool first = i0 == 0 && !split, last = i0 + n == n_fast;
      // The lanes' tree acceptance in this launch: all rows greedy, one launch.
      const bool with_accept = accept && fused && !split && n == rows;
      e = jf::launch_select_fast(F, rows_arg ? &s_rows : nullptr, n, a->dtype,
                                 uniform ? &p0 : nullptr, extras, fuse_uncut,
                                 with_accept ? accept : nullptr, accepted, stream,
                                 first ? a->select_start_event : nullptr,
                                 last ? a->select_done_event : nullptr);
    }
  }
  if (e != hipSuccess) return hip_fail((hipError_t)e, "select launch");
  // The small-K merge takes launches whose cut rows keep at most 64 tokens
  // by their top-k, or have a min-p floor (which usually leaves few: rows
  // whose floor leaves more than 64 take its general path), and read sparse
  // draft probabilities (or none).
  bool small = !staged && !a->draft_q && a->uniform_offset <= 0xffffffffull &&
               a->uniform_stride <= 0xffffffffull;
  bool wide = false;
  for (uint32_t r = 0; small && r < rows; ++r) {
    const jf::RowParams &rp = params[r];
    if ((rp.flags & jf::kRowSampled) && (rp.flags & kCuts) &&
        !((rp.flags & jf::kRowTopK) && rp.top_k <= 64u) && !(rp.flags & jf::kRowMinP))
      small = false;
    wide |= (rp.flags & jf::kRowSampled) && (rp.flags & kCuts) && !(rp.flags & jf::kRowMinP);
  }
  if (need_merge) {
    e = small ? jf::launch_merge_small(L, a->dtype, wide, stream)
              : jf::launch_merge(L, a->dtype, stream);
    if (e != hipSuccess) return hip_fail((hipError_t)e, "merge launch");
  }
  if (staged) {
    for (uint32_t stage = jf::kStageCount1; stage <= jf::kStageLast; ++stage) {
      if (stage == jf::kStageCount1 && !need_count1) continue;
      if (stage >= jf::kStageTopK3 && stage <= jf::kStageTopKLocate && !need_topk) continue;
      if (stage >= jf::kStageMass2 && stage <= jf::kStageTopPLocate && !need_topp) continue;
      if (stage == jf::kStageDraw && !L.drafted_rows) continue;
      if (stage >= jf::kStageKeptCount && !kept) continue;
      L.stage = stage;
      e = jf::launch_stage(L, a->dtype, stream);
      if (e != hipSuccess) return hip_fail((hipError_t)e, "stage launch");
    }
  }
  if (any_uncut && !fuse_uncut) {
    // residual_kernel over the kRowLean rows, then uncut_kernel: one block
    // per row, or one per (row, chunk) when other drafted uncut rows need
    // their residual pass there. A launch with lean rows and no cut row,
    // kept token list, other drafted uncut row, or sampled row whose draw
    // would reread penalized or extra values is finished by residual_kernel
    // itself (draw): each lean row by its last chunk block, every other row
    // by one of those blocks too; no uncut_kernel launch follows.
    bool draw = n_lean && !any_cut && !a->out_kept_ids && !uncut_drafted;
    for (uint32_t r = 0; draw && r < rows; ++r) {
      const jf::RowParams &rp = params[r];
      draw = !(rp.flags & jf::kRowSampled) || (rp.flags & jf::kRowLean) ||
             (!(rp.flags & jf::kRowPenalized) && !rp.extra_count);
    }
    if (n_lean) {
      thread_local std::vector<uint32_t> lean, plain;
      lean.clear();
      plain.clear();
      for (uint32_t r = 0; r < rows; ++r) {
        if (params[r].flags & jf::kRowLean)
          lean.push_back(r);
        else if (draw)
          plain.push_back(r);
      }
      // Launches of at most kKernargRows rows (a share of each list, at
      // least one lean row in each: the lean rows' blocks draw the others).
      const uint32_t nl = (uint32_t)lean.size(), np = (uint32_t)plain.size();
      const auto share = [](uint32_t total, uint32_t i, uint32_t n) {
        return (uint32_t)((uint64_t)i * total / n);
      };
      const auto fits = [&](uint32_t n) {
        for (uint32_t i = 0; i < n; ++i)
          if (share(nl, i + 1, n) - share(nl, i, n) + share(np, i + 1, n) - share(np, i, n) >
              (uint32_t)jf::kKernargRows)
            return false;
        return true;
      };
      uint32_t n = (nl + np + jf::kKernargRows - 1) / jf::kKernargRows;
      while (!fits(n)) ++n;
      if (draw && n > nl) {
        draw = false;
        plain.clear();
      }
      const uint32_t launches = draw ? n : (nl + jf::kKernargRows - 1) / jf::kKernargRows;
      jf::LeanLaunch R;
      R.a = L;
      R.draw = draw ? 1u : 0u;
      for (uint32_t i = 0; i < launches && e == hipSuccess; ++i) {
        const uint32_t l0 = share(nl, i, launches), l1 = share(nl, i + 1, launches);
        const uint32_t p0 = draw ? share(np, i, launches) : 0u,
                       p1 = draw ? share(np, i + 1, launches) : 0u;
        // The lean rows lead row_of, the others follow.
        std::memcpy(R.row_of, lean.data() + l0, (l1 - l0) * sizeof(uint32_t));
        std::memcpy(R.row_of + (l1 - l0), plain.data() + p0, (p1 - p0) * sizeof(uint32_t));
        R.n_lean = l1 - l0;
        R.n_plain = p1 - p0;
        e = jf::launch_residual(R, a->dtype, stream);
      }
      if (e != hipSuccess) return hip_fail((hipError_t)e, "residual launch");
    }
    if (!draw) {
      e = jf::launch_uncut(L, a->dtype, uncut_drafted ? L.chunks : 1u, stream);
      if (e != hipSuccess) return hip_fail((hipError_t)e, "uncut draw launch");
    }
  }
  return JF_OK;
}

}  // namespace jf

namespace {

// Room for `rows` drafted rows' stored weights, grown on first need (the
// free of a smaller buffer waits for the kernels that use it); NULL when the
// allocation fails, and the residual pass then reads the logits.
uint32_t *sampler_lean_weights(void *ctx, uint32_t rows) {
  jf_sampler *s = (jf_sampler *)ctx;
  if (rows > s->lean_rows) {
    (void)hipFree(s->lean_weights);
    s->lean_weights = nullptr;
    s->lean_rows = 0;
    void *p = nullptr;
    if (hipMalloc(&p, (size_t)rows * s->max_chunks * jf::kChunkF32 * sizeof(uint32_t)) !=
        hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    s->lean_weights = (uint32_t *)p;
    s->lean_rows = rows;
  }
  return s->lean_weights;
}

// The sampler's row parameters, uploaded through its staging ring only when
// they differ from the last upload (stream order keeps earlier launches on
// the values they were enqueued with).
int sampler_upload(void *ctx, const jf::RowParams *params, uint32_t rows,
                   jf::RowParams *device, void *stream) {
  jf_sampler *s = (jf_sampler *)ctx;
  const size_t bytes = (size_t)rows * sizeof(jf::RowParams);
  if (s->params_valid && s->last_params.size() == rows &&
      std::memcmp(s->last_params.data(), params, bytes) == 0)
    return JF_OK;
  const int rc = s->staging.upload(device, params, bytes, (hipStream_t)stream);
  if (rc != JF_OK) return rc;
  s->last_params.assign(params, params + rows);
  s->params_valid = true;
  return JF_OK;
}

}  // namespace

extern "C" {

// A finisher's wait that gave up in an earlier call (the status word set):
// reported once as JF_ERR_DEVICE, with the packed bests, arrival counters and
// chunk summaries cleared on `stream` behind every earlier launch, so that no
// word that call left behind reaches a later one.
static int take_status(jf_sampler *s, void *stream) {
  if (!__atomic_load_n(s->status_host, __ATOMIC_ACQUIRE)) return JF_OK;
  __atomic_store_n(s->status_host, 0u, __ATOMIC_RELEASE);
  const hipStream_t st = (hipStream_t)stream;
  JF_HIP(hipMemsetAsync(s->bests, 0, (size_t)s->max_rows * s->max_chunks * sizeof(uint64_t), st),
         "greedy best clear");
  JF_HIP(hipMemsetAsync(s->counters, 0, (size_t)s->max_rows * sizeof(uint32_t), st),
         "counter clear");
  JF_HIP(hipMemsetAsync(s->partials, 0,
                        (size_t)s->max_rows * s->max_chunks * sizeof(jf::StagePartial), st),
         "chunk summary clear");
  return fail(JF_ERR_DEVICE,
              "a selection's bounded wait for a chunk result expired in an earlier call; "
              "that call's rows affected hold JF_NO_TOKEN");
}

static int sample_impl(jf_sampler *s, const jf_sample_args *a, void *stream,
                       const jf::AcceptTreeLaunch *accept, bool *accepted);

int jf_sample(jf_sampler *s, const jf_sample_args *a, void *stream) {
  if (!s || !a) return fail(JF_ERR_INVALID_ARGUMENT, "null sampler or arguments");
  int rc = check_device(s->device);
  if (rc != JF_OK) return rc;
  rc = take_status(s, stream);
  if (rc != JF_OK) return rc;
  return sample_impl(s, a, stream, nullptr, nullptr);
}

// jf_sample's body after the device and status checks.
static int sample_impl(jf_sampler *s, const jf_sample_args *a, void *stream,
                       const jf::AcceptTreeLaunch *accept, bool *accepted) {
  if (!a->rows || a->rows > s->max_rows)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid sampling batch width");
  s->epoch = s->epoch % 4095u + 1u;
  const jf::SampleScratch sc{s->params,    s->headers,      s->cands,
                             s->counters,  s->bests,        s->states,
                             s->partials,  s->max_rows,     s->max_chunks,
                             s->status_device, s->epoch,    s->wait_bound,
                             sampler_lean_weights};
  if (s->host_params.size() < a->rows) {
    try {
      s->host_params.resize(a->rows);
    } catch (const std::bad_alloc &) {
      return fail(JF_ERR_NO_MEMORY, "row parameter allocation failed");
    }
  }
  return jf::sample_core(s->vocabulary, sc, a, s->host_params.data(), sampler_upload, s,
                         stream, accept, accepted);
}

int jf_sampler_status(jf_sampler *s, void *stream) {
  if (!s) return fail(JF_ERR_INVALID_ARGUMENT, "null sampler");
  const int rc = check_device(s->device);
  if (rc != JF_OK) return rc;
  return take_status(s, stream);
}

int jf_sampler_set_wait_bound(jf_sampler *s, uint32_t reads) {
  if (!s) return fail(JF_ERR_INVALID_ARGUMENT, "null sampler");
  s->wait_bound = reads;
  return JF_OK;
}

// ---- acceptance -----------------------------------------------------------

int jf_accept_chain(jf_sampler *s, const jf_accept_chain_args *a,
                    void *stream) {
  if (!s || !a) return fail(JF_ERR_INVALID_ARGUMENT, "null sampler or arguments");
  int rc = check_device(s->device);
  if (rc != JF_OK) return rc;
  if (!a->lanes || a->lanes > s->max_rows || !a->maximum_retained || !a->policies)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid DFlash acceptance batch");
  if (a->verify_rows != 8 && a->verify_rows != 16)
    return fail(JF_ERR_INVALID_ARGUMENT, "verify shape must be 8 or 16");
  if (!a->proposed_tokens || !a->target_tokens || !a->retained_counts ||
      !a->accepted_counts)
    return fail(JF_ERR_INVALID_ARGUMENT, "null acceptance buffer");
  bool any_sampled = false;
  for (uint32_t l = 0; l < a->lanes; ++l) {
    const uint32_t m = a->maximum_retained[l];
    if (!m || m > a->verify_rows)
      return fail(JF_ERR_INVALID_ARGUMENT, "invalid DFlash retention limit");
    any_sampled |= a->policies[l].temperature > 0.0f;
  }
  if (any_sampled && (!a->candidates || !a->proposal_probs ||
                      !a->target_draft_probs || !a->uniforms))
    return fail(JF_ERR_INVALID_ARGUMENT, "sampled acceptance needs candidates, "
                                         "probabilities and uniforms");
  // The lanes' records travel in the kernel arguments, kChainLanesPerLaunch
  // lanes a launch: nothing is uploaded.
  const uint32_t P = a->verify_rows - 1;
  jf::AcceptChainLaunch L;
  L.verify_rows = a->verify_rows;
  L.stop0 = a->stop_token_0;
  L.stop1 = a->stop_token_1;
  for (uint32_t l0 = 0; l0 < a->lanes; l0 += jf::kChainLanesPerLaunch) {
    const uint32_t n = std::min(a->lanes - l0, jf::kChainLanesPerLaunch);
    L.lanes = n;
    L.proposed = a->proposed_tokens + (uint64_t)l0 * P;
    L.candidates = a->candidates ? a->candidates + (uint64_t)l0 * P * 16 : nullptr;
    L.proposal_probs = a->proposal_probs ? a->proposal_probs + (uint64_t)l0 * P * 16 : nullptr;
    L.target_draft_probs =
        a->target_draft_probs ? a->target_draft_probs + (uint64_t)l0 * a->verify_rows : nullptr;
    L.uniforms = a->uniforms ? a->uniforms + (uint64_t)l0 * 40 : nullptr;
    L.target_tokens = a->target_tokens + (uint64_t)l0 * a->verify_rows;
    L.retained = a->retained_counts + l0;
    L.accepted = a->accepted_counts + l0;
    for (uint32_t i = 0; i < n; ++i) {
      L.lane_params[i].remaining = a->maximum_retained[l0 + i];
      L.lane_params[i].sampled = a->policies[l0 + i].temperature > 0.0f ? 1u : 0u;
    }
    const int e = jf::launch_accept_chain(L, stream);
    if (e != hipSuccess) return hip_fail((hipError_t)e, "acceptance launch");
  }
  return JF_OK;
}

// Checks a tree acceptance call (any_sampled: some lane samples).
static int check_tree_args(jf_sampler *s, const jf_accept_tree_args *a, bool *any_sampled) {
  if (!a->lanes || a->lanes > s->max_rows || !a->trees || !a->maximum_retained ||
      !a->policies)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid tree acceptance batch");
  if (!a->rows_per_lane || a->rows_per_lane > JF_TREE_MAXIMUM_ROWS)
    return fail(JF_ERR_INVALID_ARGUMENT, "tree rows per lane must be 1..16");
  if (!a->target_tokens || !a->retained_counts || !a->accepted_counts ||
      !a->path_rows)
    return fail(JF_ERR_INVALID_ARGUMENT, "null acceptance buffer");
  *any_sampled = false;
  for (uint32_t l = 0; l < a->lanes; ++l) {
    const jf_tree_lane &t = a->trees[l];
    if (!t.rows || t.rows > a->rows_per_lane || t.chain_rows > t.rows)
      return fail(JF_ERR_INVALID_ARGUMENT, "invalid draft tree rows");
    for (uint32_t r = 1; r < t.rows; ++r)
      if (t.parent[r] >= r)
        return fail(JF_ERR_INVALID_ARGUMENT, "draft tree rows are not in DFS preorder");
    // Rows 0 .. chain_rows - 1 are the draft's sampled chain (each the
    // previous row's child): the walk reads chain_q at those rows only.
    for (uint32_t r = 1; r < t.chain_rows; ++r)
      if (t.parent[r] != r - 1)
        return fail(JF_ERR_INVALID_ARGUMENT, "draft tree chain rows do not form a chain");
    const uint32_t m = a->maximum_retained[l];
    if (!m || m > JF_TREE_MAXIMUM_DEPTH)
      return fail(JF_ERR_INVALID_ARGUMENT, "invalid tree retention limit");
    *any_sampled |= a->policies[l].temperature > 0.0f;
  }
  if (*any_sampled && (!a->target_draft_probs || !a->uniforms))
    return fail(JF_ERR_INVALID_ARGUMENT,
                "sampled tree acceptance needs probabilities and uniforms");
  return JF_OK;
}

// The launch record of lanes l0 .. l0 + n - 1 (n <= kTreeLanesPerLaunch):
// their trees travel in the kernel arguments, nothing is uploaded.
static void fill_tree_launch(const jf_accept_tree_args *a, uint32_t l0, uint32_t n,
                             jf::AcceptTreeLaunch &L) {
  const uint32_t R = a->rows_per_lane;
  L.rows_per_lane = R;
  L.stop0 = a->stop_token_0;
  L.stop1 = a->stop_token_1;
  L.lanes = n;
  L.target_draft_probs =
      a->target_draft_probs ? a->target_draft_probs + (uint64_t)l0 * R : nullptr;
  L.uniforms = a->uniforms ? a->uniforms + (uint64_t)l0 * 40 : nullptr;
  L.target_tokens = a->target_tokens + (uint64_t)l0 * R;
  L.retained = a->retained_counts + l0;
  L.accepted = a->accepted_counts + l0;
  L.path_rows = a->path_rows + (uint64_t)l0 * 8;
  for (uint32_t i = 0; i < n; ++i) {
    const jf_tree_lane &t = a->trees[l0 + i];
    jf::TreeLaneParams &p = L.trees[i];
    p.rows = t.rows;
    p.chain_rows = t.chain_rows;
    p.remaining = a->maximum_retained[l0 + i];
    p.sampled = a->policies[l0 + i].temperature > 0.0f ? 1u : 0u;
    std::memcpy(p.parent, t.parent, sizeof(p.parent));
    std::memcpy(p.token, t.token, sizeof(p.token));
    std::memcpy(p.chain_q, t.chain_q, sizeof(p.chain_q));
  }
}

static int accept_tree_checked(const jf_accept_tree_args *a, void *stream) {
  jf::AcceptTreeLaunch L;
  for (uint32_t l0 = 0; l0 < a->lanes; l0 += jf::kTreeLanesPerLaunch) {
    fill_tree_launch(a, l0, std::min(a->lanes - l0, jf::kTreeLanesPerLaunch), L);
    const int e = jf::launch_accept_tree(L, stream);
    if (e != hipSuccess) return hip_fail((hipError_t)e, "tree acceptance launch");
  }
  return JF_OK;
}

int jf_accept_tree(jf_sampler *s, const jf_accept_tree_args *a, void *stream) {
  if (!s || !a) return fail(JF_ERR_INVALID_ARGUMENT, "null sampler or arguments");
  int rc = check_device(s->device);
  if (rc != JF_OK) return rc;
  bool any_sampled;
  rc = check_tree_args(s, a, &any_sampled);
  if (rc != JF_OK) return rc;
  return accept_tree_checked(a, stream);
}

int jf_sample_accept_tree(jf_sampler *s, const jf_sample_args *sa,
                          const jf_accept_tree_args *ta, void *stream) {
  if (!s || !sa || !ta) return fail(JF_ERR_INVALID_ARGUMENT, "null sampler or arguments");
  int rc = check_device(s->device);
  if (rc != JF_OK) return rc;
  rc = take_status(s, stream);
  if (rc != JF_OK) return rc;
  bool any_sampled;
  rc = check_tree_args(s, ta, &any_sampled);
  if (rc != JF_OK) return rc;
  // In the selection's launch when the lanes are greedy, take the
  // selection's rows in order and fit one launch record.
  const bool fusable = !any_sampled && ta->lanes <= jf::kTreeLanesPerLaunch &&
                       (uint64_t)ta->lanes * ta->rows_per_lane == sa->rows &&
                       ta->target_tokens == sa->out_tokens;
  jf::AcceptTreeLaunch L;
  if (fusable) fill_tree_launch(ta, 0, ta->lanes, L);
  bool accepted = false;
  rc = sample_impl(s, sa, stream, fusable ? &L : nullptr, &accepted);
  if (rc != JF_OK) return rc;
  return accepted ? JF_OK : accept_tree_checked(ta, stream);
}

// ---- draft selector ----------------------------------------------------------

}  // extern "C"

struct jf_draft_selector {
  uint32_t vocabulary = 0;
  uint32_t max_lanes = 0;
  uint32_t chunks = 0;
  int device = 0;
  jf::DraftLaneParams *lane_params = nullptr;  // [max_lanes]
  uint64_t *part_comp = nullptr;               // [max_lanes * 7][chunks][16]
  uint32_t *part_vbits = nullptr;
  float *tables = nullptr;                     // [max_lanes][7][16][16]
  uint32_t *choices = nullptr;                 // [max_lanes * 7][16]
  float *choice_q = nullptr;                   // [max_lanes * 7][16][16]
  uint32_t *counters = nullptr;                // [max_lanes * 8]
  std::vector<jf::DraftLaneParams> last_lanes;  // what lane_params holds
  StagingRing staging;
};

extern "C" {

int jf_draft_selector_destroy(jf_draft_selector *d) {
  if (!d) return JF_OK;
  d->staging.release();
  (void)hipFree(d->lane_params);
  (void)hipFree(d->part_comp);
  (void)hipFree(d->part_vbits);
  (void)hipFree(d->tables);
  (void)hipFree(d->choices);
  (void)hipFree(d->choice_q);
  (void)hipFree(d->counters);
  delete d;
  return JF_OK;
}

int jf_draft_selector_create(uint32_t vocabulary, uint32_t max_lanes,
                             jf_draft_selector **out) {
  if (!out) return fail(JF_ERR_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  // DraftSelector.cpp:22-25 and DraftSelector::workspace (27-36).
  if (!vocabulary) return fail(JF_ERR_INVALID_ARGUMENT, "invalid draft selector vocabulary");
  if (!max_lanes)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid draft selector workspace position count");
  const uint32_t chunks = (vocabulary + 8191u) / 8192u;
  if (chunks > 64) return fail(JF_ERR_INVALID_ARGUMENT, "vocabulary exceeds 524288 tokens");
  jf_draft_selector *d = new (std::nothrow) jf_draft_selector;
  if (!d) return fail(JF_ERR_NO_MEMORY, "draft selector allocation failed");
  d->vocabulary = vocabulary;
  d->max_lanes = max_lanes;
  d->chunks = chunks;
  int rc = JF_OK;
  const hipError_t ge = hipGetDevice(&d->device);
  if (ge != hipSuccess) rc = hip_fail(ge, "hipGetDevice");
  const uint64_t rows = (uint64_t)max_lanes * jf::kDraftPositions;
  if (rc == JF_OK) rc = device_alloc(&d->lane_params, max_lanes, "draft lane parameters");
  if (rc == JF_OK) rc = device_alloc(&d->part_comp, rows * chunks * JF_DRAFT_CANDIDATES, "draft partials");
  if (rc == JF_OK) rc = device_alloc(&d->part_vbits, rows * chunks * JF_DRAFT_CANDIDATES, "draft partial values");
  if (rc == JF_OK)
    rc = device_alloc(&d->tables, rows * JF_DRAFT_CANDIDATES * JF_DRAFT_CANDIDATES, "draft edge tables");
  if (rc == JF_OK) rc = device_alloc(&d->choices, rows * JF_DRAFT_CANDIDATES, "draft walk choices");
  if (rc == JF_OK)
    rc = device_alloc(&d->choice_q, rows * JF_DRAFT_CANDIDATES * JF_DRAFT_CANDIDATES,
                      "draft walk probabilities");
  if (rc == JF_OK) rc = device_alloc(&d->counters, (uint64_t)max_lanes * jf::kDraftQueryRows, "draft counters");
  if (rc == JF_OK) {
    const hipError_t e1 = hipMemset(d->counters, 0, (uint64_t)max_lanes * jf::kDraftQueryRows * sizeof(uint32_t));
    const hipError_t e2 = hipDeviceSynchronize();
    if (e1 != hipSuccess) rc = hip_fail(e1, "counter init");
    else if (e2 != hipSuccess) rc = hip_fail(e2, "init sync");
  }
  if (rc != JF_OK) {
    jf_draft_selector_destroy(d);
    return rc;
  }
  *out = d;
  return JF_OK;
}

int jf_draft_select(jf_draft_selector *d, const jf_draft_select_args *a, void *stream) {
  if (!d || !a) return fail(JF_ERR_INVALID_ARGUMENT, "null selector or arguments");
  int rc = check_device(d->device);
  if (rc != JF_OK) return rc;
  // DraftSelector::add's checks (DraftSelector.cpp:43-76), before any launch.
  if (!a->lanes || a->lanes > d->max_lanes || !a->anchors || !a->policies)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid draft selector batch");
  if (!a->logits || a->logits_stride < d->vocabulary)
    return fail(JF_ERR_INVALID_ARGUMENT, "draft logits buffer too small");
  if (!a->selector_hidden) return fail(JF_ERR_INVALID_ARGUMENT, "draft selector hidden buffer too small");
  if (!a->predecessor_codebook || !a->successor_codebook ||
      (uintptr_t)a->predecessor_codebook % 16 || (uintptr_t)a->successor_codebook % 16)
    return fail(JF_ERR_INVALID_ARGUMENT, "draft codebooks must be 16-byte aligned device buffers");
  if (!a->candidates || !a->unary || !a->proposed_tokens)
    return fail(JF_ERR_INVALID_ARGUMENT, "draft candidate buffer too small");
  if ((a->select_start_event == nullptr) != (a->select_done_event == nullptr))
    return fail(JF_ERR_INVALID_ARGUMENT, "select events come in pairs");
  std::vector<jf::DraftLaneParams> lanes(a->lanes);
  bool any_sampled = false;
  for (uint32_t l = 0; l < a->lanes; ++l) {
    const float t = a->policies[l].temperature;
    if (!(t == 0.0f || (std::isfinite(t) && t >= FLT_MIN)))
      return fail(JF_ERR_INVALID_ARGUMENT,
                  "sampling requires temperature 0 or at least FLT_MIN, top_p in (0,1] and "
                  "min_p in [0,1]");
    lanes[l].anchor = a->anchors[l];
    lanes[l].temperature = t;
    lanes[l].sampled = t > 0.0f ? 1u : 0u;
    any_sampled |= t > 0.0f;
  }
  if (any_sampled && (!a->uniforms || !a->proposal_probs))
    return fail(JF_ERR_INVALID_ARGUMENT, "proposal uniform buffer too small");
  // Uploaded only when they change (stream order keeps earlier launches on
  // the values they were enqueued with).
  const size_t lane_bytes = lanes.size() * sizeof(jf::DraftLaneParams);
  if (d->last_lanes.size() != lanes.size() ||
      std::memcmp(d->last_lanes.data(), lanes.data(), lane_bytes) != 0) {
    d->last_lanes.clear();
    rc = d->staging.upload(d->lane_params, lanes.data(), lane_bytes, (hipStream_t)stream);
    if (rc != JF_OK) return rc;
    d->last_lanes = lanes;
  }
  jf::DraftLaunch L{};
  L.logits = a->logits;
  L.stride = a->logits_stride;
  L.vocabulary = d->vocabulary;
  L.chunks = d->chunks;
  L.lanes = a->lanes;
  L.hidden = a->selector_hidden;
  L.pred_codebook = a->predecessor_codebook;
  L.succ_codebook = a->successor_codebook;
  L.lane_params = d->lane_params;
  L.uniforms = a->uniforms;
  L.candidates = a->candidates;
  L.unary = a->unary;
  L.tokens = a->proposed_tokens;
  L.q_probs = a->proposal_probs;
  L.part_comp = d->part_comp;
  L.part_vbits = d->part_vbits;
  L.tables = a->edge_tables ? a->edge_tables : d->tables;
  L.choices = d->choices;
  L.choice_q = d->choice_q;
  L.counters = d->counters;
  const bool aligned = (uintptr_t)a->logits % 16 == 0 && a->logits_stride % 4 == 0;
  const int e = jf::launch_draft_select(L, aligned, stream, a->select_start_event,
                                        a->select_done_event);
  if (e != hipSuccess) return hip_fail((hipError_t)e, "draft selector launch");
  return JF_OK;
}

// ---- tree gather -------------------------------------------------------------

int jf_tree_gather(const jf_tree_gather_args *a, void *stream) {
  if (!a) return fail(JF_ERR_INVALID_ARGUMENT, "null tree gather arguments");
  if (!a->data || !a->path_rows || !a->retained)
    return fail(JF_ERR_INVALID_ARGUMENT, "tree gather buffers are null");
  if (!a->columns || !a->inner || !a->layers || !a->lanes || !a->rows ||
      a->rows > JF_TREE_MAXIMUM_ROWS)
    return fail(JF_ERR_INVALID_ARGUMENT, "invalid tree gather geometry");
  if ((a->start_event == nullptr) != (a->done_event == nullptr))
    return fail(JF_ERR_INVALID_ARGUMENT, "gather events come in pairs");
  // The largest unit any thread touches.
  const uint64_t last_column = a->columns - 1u;
  const uint64_t in_group = std::min<uint64_t>(a->inner - 1u, last_column);
  const uint64_t top = (uint64_t)(a->layers - 1u) * a->layer_stride +
                       (uint64_t)(a->lanes - 1u) * a->lane_stride +
                       (uint64_t)(a->rows - 1u) * a->row_stride +
                       (last_column / a->inner) * a->outer_stride + in_group * a->inner_stride;
  if (top >= a->data_units) return fail(JF_ERR_INVALID_ARGUMENT, "tree gather data buffer too small");
  jf::GatherLaunch g{};
  g.data = a->data;
  g.path_rows = a->path_rows;
  g.retained = a->retained;
  g.columns = a->columns;
  g.inner = a->inner;
  g.inner_stride = a->inner_stride;
  g.outer_stride = a->outer_stride;
  g.row_stride = a->row_stride;
  g.lane_stride = a->lane_stride;
  g.layer_stride = a->layer_stride;
  g.layers = a->layers;
  g.lanes = a->lanes;
  g.rows = a->rows;
  // 8 columns a thread when a row's columns are contiguous 16-byte runs.
  const bool vec8 = (uintptr_t)a->data % 16 == 0 && a->inner_stride == 1 && a->inner % 8 == 0 &&
                    a->columns % 8 == 0 && a->outer_stride % 8 == 0 && a->row_stride % 8 == 0 &&
                    a->row_stride >= 8 && a->lane_stride % 8 == 0 && a->layer_stride % 8 == 0;
  const int e = jf::launch_tree_gather(g, vec8, stream, a->start_event, a->done_event);
  if (e != hipSuccess) return hip_fail((hipError_t)e, "tree gather launch");
  return JF_OK;
}

}  // extern "C"
