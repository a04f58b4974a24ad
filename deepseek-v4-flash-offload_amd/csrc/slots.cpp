// Expert slot cache: host pool of packed experts + LRU of device slots.
//
// Replaces the ExpertBank device caches of offload.py:86-129 (OrderedDict LRU,
// per-expert `.to(device, non_blocking=True)` on the compute stream, fresh
// allocations per miss) with:
//   * one device slot pool (borrowed from the caller, n_slots x record_bytes),
//     each slot holding one expert's six packed tensors at fixed offsets;
//   * pinned host records (hipHostMalloc, allocated in chunks) holding the same
//     bytes, so a miss is ONE contiguous hipMemcpyAsync of the whole expert;
//   * a side copy stream: misses are copied there while the compute stream keeps
//     running earlier layers; the compute stream waits on one event per batch;
//   * slot reuse ordered by events: before a victim slot is overwritten, the
//     copy stream waits for the compute work that last read it.
// The LRU policy is the reference's: a hit moves the key to the MRU end, a miss
// takes a free slot or evicts the least recently used key.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "../../include/dsv4_moe.h"

int dsv4_fail(int code, const char* fmt, ...);

namespace {

// ---------------------------------------------------------------------------
// LRU over a fixed number of slots (host only).
// ---------------------------------------------------------------------------
class SlotLRU {
 public:
  explicit SlotLRU(int n) : n_(n), key_(n, -1), prev_(n, -1), next_(n, -1), mark_(n, 0) {
    for (int s = n - 1; s >= 0; --s) free_.push_back(s);
  }
  int capacity() const { return n_; }
  int size() const { return (int)map_.size(); }

  // Returns 1 on hit, 0 on miss, -1 if every slot is marked by the current batch.
  int access(int64_t key, uint32_t batch_mark, int* slot, int64_t* evicted) {
    *evicted = -1;
    auto it = map_.find(key);
    if (it != map_.end()) {
      const int s = it->second;
      unlink(s);
      push_mru(s);
      mark_[s] = batch_mark;
      *slot = s;
      return 1;
    }
    int s;
    if (!free_.empty()) {
      s = free_.back();
      free_.pop_back();
    } else {
      s = lru_;
      while (s >= 0 && mark_[s] == batch_mark && batch_mark != 0) s = next_[s];
      if (s < 0) return -1;
      unlink(s);
      map_.erase(key_[s]);
      *evicted = key_[s];
    }
    key_[s] = key;
    map_[key] = s;
    push_mru(s);
    mark_[s] = batch_mark;
    *slot = s;
    return 0;
  }

  bool lookup(int64_t key, int* slot) const {
    auto it = map_.find(key);
    if (it == map_.end()) return false;
    *slot = it->second;
    return true;
  }

  // keys from least to most recently used
  int keys(int64_t* out, int max) const {
    int c = 0;
    for (int s = lru_; s >= 0 && c < max; s = next_[s]) out[c++] = key_[s];
    return c;
  }

  void clear() {
    map_.clear();
    free_.clear();
    for (int s = n_ - 1; s >= 0; --s) {
      free_.push_back(s);
      key_[s] = -1;
      prev_[s] = next_[s] = -1;
      mark_[s] = 0;
    }
    lru_ = mru_ = -1;
  }

 private:
  void unlink(int s) {
    if (prev_[s] >= 0) next_[prev_[s]] = next_[s]; else lru_ = next_[s];
    if (next_[s] >= 0) prev_[next_[s]] = prev_[s]; else mru_ = prev_[s];
    prev_[s] = next_[s] = -1;
  }
  void push_mru(int s) {
    prev_[s] = mru_;
    next_[s] = -1;
    if (mru_ >= 0) next_[mru_] = s; else lru_ = s;
    mru_ = s;
  }
  int n_;
  std::vector<int64_t> key_;
  std::vector<int> prev_, next_;  // prev = towards LRU, next = towards MRU
  std::vector<uint32_t> mark_;
  std::vector<int> free_;
  std::unordered_map<int64_t, int> map_;
  int lru_ = -1, mru_ = -1;
};

inline int64_t make_key(int layer, int eid) { return ((int64_t)(uint32_t)layer << 32) | (uint32_t)eid; }

constexpr int kRing = 256;

}  // namespace

// ---------------------------------------------------------------------------
struct dsv4_slots {
  int device = 0;
  int64_t record_bytes = 0;
  int n_slots = 0;
  uint8_t* pool = nullptr;  // borrowed device memory
  SlotLRU lru{0};
  hipStream_t copy_stream = nullptr;
  hipEvent_t copy_ev[kRing];
  hipEvent_t rel_ev[kRing];
  int64_t copy_seq = 0;     // number of copy batches recorded
  int64_t rel_seq = 0;      // number of releases recorded
  std::vector<int64_t> slot_copy_seq;  // 1-based batch id of the slot's pending/last copy (0 = none)
  std::vector<int64_t> slot_rel_seq;   // 1-based release id of the slot's last reader (0 = none)
  std::vector<int> last_used;          // slots of the last acquire
  uint32_t batch_mark = 0;
  // host records
  bool pinned = true;
  int64_t records_per_chunk = 0;
  std::vector<uint8_t*> chunks;
  std::vector<bool> chunk_pinned;
  int64_t chunk_fill = 0;  // records used in the last chunk
  std::unordered_map<int64_t, uint8_t*> records;
  // counters
  int64_t hits = 0, misses = 0, evictions = 0, prefetched = 0, bytes_h2d = 0, copies = 0;
  std::mutex mu;
  explicit dsv4_slots(int n) : lru(n) {}
};

#define SREQ(cond, code, ...) \
  do {                        \
    if (!(cond)) return dsv4_fail(code, __VA_ARGS__); \
  } while (0)
#define SHIP(call)                                                                         \
  do {                                                                                     \
    hipError_t _e = (call);                                                                \
    if (_e != hipSuccess) return dsv4_fail(DSV4_ERR_HIP, "%s: %s", #call, hipGetErrorString(_e)); \
  } while (0)

extern "C" {

// ----------------------------- LRU core (host only) ------------------------
int dsv4_lru_create(int capacity, void** out) {
  SREQ(out, DSV4_ERR_NULL, "lru: null output");
  SREQ(capacity >= 0, DSV4_ERR_SHAPE, "lru: negative capacity");
  *out = new SlotLRU(capacity);
  return DSV4_OK;
}
int dsv4_lru_destroy(void* h) {
  delete (SlotLRU*)h;
  return DSV4_OK;
}
int dsv4_lru_access(void* h, int64_t key, int* hit, int* slot, int64_t* evicted) {
  SREQ(h && hit && slot && evicted, DSV4_ERR_NULL, "lru: null pointer");
  SlotLRU* l = (SlotLRU*)h;
  if (l->capacity() == 0) {  // capacity 0 never caches (offload.py:95)
    *hit = 0;
    *slot = -1;
    *evicted = -1;
    return DSV4_OK;
  }
  int r = l->access(key, 0, slot, evicted);
  *hit = r;
  return DSV4_OK;
}
int dsv4_lru_keys(void* h, int64_t* out, int max, int* n) {
  SREQ(h && out && n, DSV4_ERR_NULL, "lru: null pointer");
  *n = ((SlotLRU*)h)->keys(out, max);
  return DSV4_OK;
}

// ----------------------------- slot manager --------------------------------
int dsv4_slots_create(int device, int64_t record_bytes, int n_slots, void* device_pool, int pin_host,
                      dsv4_slots** out) {
  SREQ(out, DSV4_ERR_NULL, "slots: null output");
  SREQ(record_bytes > 0 && record_bytes % 256 == 0, DSV4_ERR_SHAPE,
       "slots: record_bytes %lld must be a positive multiple of 256", (long long)record_bytes);
  SREQ(n_slots > 0, DSV4_ERR_SHAPE, "slots: need at least one slot");
  SREQ(device_pool && ((uintptr_t)device_pool % 256) == 0, DSV4_ERR_NULL, "slots: device pool null or misaligned");
  SHIP(hipSetDevice(device));
  dsv4_slots* s = new dsv4_slots(n_slots);
  s->device = device;
  s->record_bytes = record_bytes;
  s->n_slots = n_slots;
  s->pool = (uint8_t*)device_pool;
  s->pinned = pin_host != 0;
  s->records_per_chunk = record_bytes >= (int64_t)1 << 30 ? 1 : (((int64_t)1 << 30) / record_bytes);
  s->slot_copy_seq.assign(n_slots, 0);
  s->slot_rel_seq.assign(n_slots, 0);
  hipError_t e = hipStreamCreateWithFlags(&s->copy_stream, hipStreamNonBlocking);
  for (int i = 0; i < kRing && e == hipSuccess; ++i) {
    e = hipEventCreateWithFlags(&s->copy_ev[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s->rel_ev[i], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    delete s;
    return dsv4_fail(DSV4_ERR_HIP, "slots: stream/event creation: %s", hipGetErrorString(e));
  }
  *out = s;
  return DSV4_OK;
}

int dsv4_slots_destroy(dsv4_slots* s) {
  if (!s) return DSV4_OK;
  // best effort teardown: errors here have no caller to report to
  (void)hipSetDevice(s->device);
  if (s->copy_stream) (void)hipStreamSynchronize(s->copy_stream);
  for (int i = 0; i < kRing; ++i) {
    (void)hipEventDestroy(s->copy_ev[i]);
    (void)hipEventDestroy(s->rel_ev[i]);
  }
  if (s->copy_stream) (void)hipStreamDestroy(s->copy_stream);
  for (size_t i = 0; i < s->chunks.size(); ++i) {
    if (s->chunk_pinned[i]) (void)hipHostFree(s->chunks[i]); else free(s->chunks[i]);
  }
  delete s;
  return DSV4_OK;
}

// Host record of (layer, eid), allocated on first use. *pinned_out tells whether
// the record is page-locked (1) or pageable after a failed pinned allocation (0).
int dsv4_slots_host_record(dsv4_slots* s, int layer, int eid, int create, void** rec, int* pinned_out) {
  SREQ(s && rec, DSV4_ERR_NULL, "slots: null pointer");
  std::lock_guard<std::mutex> g(s->mu);
  const int64_t key = make_key(layer, eid);
  auto it = s->records.find(key);
  if (it != s->records.end()) {
    *rec = it->second;
  } else {
    SREQ(create, DSV4_ERR_STATE, "slots: expert (%d, %d) is not registered", layer, eid);
    if (s->chunks.empty() || s->chunk_fill == s->records_per_chunk) {
      const size_t bytes = (size_t)(s->records_per_chunk * s->record_bytes);
      void* p = nullptr;
      bool pinned = false;
      if (s->pinned) {
        SHIP(hipSetDevice(s->device));
        if (hipHostMalloc(&p, bytes, hipHostMallocDefault) == hipSuccess) pinned = true;
        else { (void)hipGetLastError(); p = nullptr; s->pinned = false; }
      }
      if (!p) p = aligned_alloc(256, bytes);
      SREQ(p, DSV4_ERR_STATE, "slots: host allocation of %zu bytes failed", bytes);
      s->chunks.push_back((uint8_t*)p);
      s->chunk_pinned.push_back(pinned);
      s->chunk_fill = 0;
    }
    uint8_t* r = s->chunks.back() + s->chunk_fill * s->record_bytes;
    ++s->chunk_fill;
    s->records[key] = r;
    *rec = r;
  }
  if (pinned_out) {
    *pinned_out = 0;
    const uint8_t* r = (const uint8_t*)*rec;
    for (size_t i = 0; i < s->chunks.size(); ++i)
      if (r >= s->chunks[i] && r < s->chunks[i] + s->records_per_chunk * s->record_bytes)
        *pinned_out = s->chunk_pinned[i] ? 1 : 0;
  }
  return DSV4_OK;
}

int dsv4_slots_num_registered(dsv4_slots* s, int64_t* n) {
  SREQ(s && n, DSV4_ERR_NULL, "slots: null pointer");
  std::lock_guard<std::mutex> g(s->mu);
  *n = (int64_t)s->records.size();
  return DSV4_OK;
}

// Shared body of acquire/prefetch. For acquire, the compute stream is made to
// wait for every copy the returned slots depend on.
// Records the release event of the previous acquire's slots on `compute`: every
// read of those slots enqueued on `compute` so far is ordered before any later
// copy into them. Caller holds the mutex.
static int release_locked(dsv4_slots* s, hipStream_t compute) {
  if (s->last_used.empty()) return DSV4_OK;
  const int64_t seq = ++s->rel_seq;
  SHIP(hipEventRecord(s->rel_ev[(seq - 1) % kRing], compute));
  for (int slot : s->last_used) s->slot_rel_seq[slot] = seq;
  s->last_used.clear();
  return DSV4_OK;
}

static int slots_fetch(dsv4_slots* s, int layer, const int32_t* eids, int n, hipStream_t compute, bool is_acquire,
                       int32_t* slots_out, int* n_miss) {
  SREQ(s && (n == 0 || eids), DSV4_ERR_NULL, "slots: null pointer");
  SREQ(n >= 0 && n <= s->n_slots, DSV4_ERR_SHAPE, "slots: batch of %d experts exceeds %d slots", n, s->n_slots);
  std::lock_guard<std::mutex> g(s->mu);
  SHIP(hipSetDevice(s->device));
  if (is_acquire) {
    // the slots handed out by the previous acquire stay valid for work enqueued
    // on the compute stream up to this call (release-at-next-acquire)
    int rc = release_locked(s, compute);
    if (rc) return rc;
  }
  // An acquire starts a new batch. A prefetch joins the current one: the slots
  // the last acquire handed out are still to be read by work the caller has not
  // enqueued yet (their release is recorded only at the next acquire), so they
  // must not become a prefetch's victims.
  const uint32_t mark =
      is_acquire ? (++s->batch_mark == 0 ? ++s->batch_mark : s->batch_mark) : s->batch_mark;
  int64_t wait_seq = 0;
  bool issued = false;
  int misses = 0;
  const int64_t this_seq = s->copy_seq + 1;
  for (int i = 0; i < n; ++i) {
    const int64_t key = make_key(layer, eids[i]);
    auto rit = s->records.find(key);
    SREQ(rit != s->records.end(), DSV4_ERR_STATE, "slots: expert (%d, %d) is not registered", layer, eids[i]);
    int slot;
    int64_t evicted;
    if (!is_acquire) {
      int tmp;
      if (s->lru.lookup(key, &tmp)) continue;  // already resident or in flight: leave recency alone
    }
    const int r = s->lru.access(key, mark, &slot, &evicted);
    if (r < 0 && !is_acquire) break;  // a prefetch is advisory: stop when only pinned slots are left
    SREQ(r >= 0, DSV4_ERR_STATE, "slots: all %d slots are pinned by this batch", s->n_slots);
    if (r == 1) {
      if (is_acquire) ++s->hits;
      if (s->slot_copy_seq[slot] > wait_seq) wait_seq = s->slot_copy_seq[slot];
    } else {
      ++misses;
      if (is_acquire) ++s->misses; else ++s->prefetched;
      if (evicted >= 0) ++s->evictions;
      if (s->slot_rel_seq[slot] > 0)  // the slot's last reader must finish before it is overwritten
        SHIP(hipStreamWaitEvent(s->copy_stream, s->rel_ev[(s->slot_rel_seq[slot] - 1) % kRing], 0));
      SHIP(hipMemcpyAsync(s->pool + (int64_t)slot * s->record_bytes, rit->second, (size_t)s->record_bytes,
                          hipMemcpyHostToDevice, s->copy_stream));
      s->bytes_h2d += s->record_bytes;
      ++s->copies;
      s->slot_copy_seq[slot] = this_seq;
      wait_seq = this_seq;
      issued = true;
    }
    if (slots_out) slots_out[i] = slot;
    if (is_acquire) s->last_used.push_back(slot);
  }
  if (issued) {
    SHIP(hipEventRecord(s->copy_ev[(this_seq - 1) % kRing], s->copy_stream));
    s->copy_seq = this_seq;
  }
  if (is_acquire && wait_seq > 0) SHIP(hipStreamWaitEvent(compute, s->copy_ev[(wait_seq - 1) % kRing], 0));
  if (n_miss) *n_miss = misses;
  return DSV4_OK;
}

int dsv4_slots_acquire(dsv4_slots* s, int layer, const int32_t* eids, int n, void* compute_stream,
                       int32_t* slots_out, int* n_miss) {
  SREQ(slots_out || n == 0, DSV4_ERR_NULL, "slots: null slot output");
  return slots_fetch(s, layer, eids, n, (hipStream_t)compute_stream, true, slots_out, n_miss);
}

int dsv4_slots_prefetch(dsv4_slots* s, int layer, const int32_t* eids, int n, int* n_issued) {
  return slots_fetch(s, layer, eids, n, nullptr, false, nullptr, n_issued);
}

int dsv4_slots_release(dsv4_slots* s, void* compute_stream) {
  SREQ(s, DSV4_ERR_NULL, "slots: null handle");
  std::lock_guard<std::mutex> g(s->mu);
  SHIP(hipSetDevice(s->device));
  return release_locked(s, (hipStream_t)compute_stream);
}

// Copies the host record of (layer, eid) to `dst` (device, record_bytes) on
// `stream`, outside the slot cache (the reference's per-miss H2D of get()).
int dsv4_slots_copy_record(dsv4_slots* s, int layer, int eid, void* dst, void* stream) {
  SREQ(s && dst, DSV4_ERR_NULL, "slots: null pointer");
  std::lock_guard<std::mutex> g(s->mu);
  auto it = s->records.find(make_key(layer, eid));
  SREQ(it != s->records.end(), DSV4_ERR_STATE, "slots: expert (%d, %d) is not registered", layer, eid);
  SHIP(hipSetDevice(s->device));
  SHIP(hipMemcpyAsync(dst, it->second, (size_t)s->record_bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
  return DSV4_OK;
}

int dsv4_slots_lookup(dsv4_slots* s, int layer, int eid, int32_t* slot) {
  SREQ(s && slot, DSV4_ERR_NULL, "slots: null pointer");
  std::lock_guard<std::mutex> g(s->mu);
  int sl;
  *slot = s->lru.lookup(make_key(layer, eid), &sl) ? sl : -1;
  return DSV4_OK;
}

int dsv4_slots_keys(dsv4_slots* s, int64_t* out, int max, int* n) {
  SREQ(s && out && n, DSV4_ERR_NULL, "slots: null pointer");
  std::lock_guard<std::mutex> g(s->mu);
  *n = s->lru.keys(out, max);
  return DSV4_OK;
}

int dsv4_slots_sync(dsv4_slots* s) {
  SREQ(s, DSV4_ERR_NULL, "slots: null handle");
  SHIP(hipSetDevice(s->device));
  SHIP(hipStreamSynchronize(s->copy_stream));
  return DSV4_OK;
}

// Forgets every resident expert (offload.py:131-133 drops its cached dicts).
// The slots of the last acquire may still be read by work the caller enqueued on
// `compute_stream`: their release is recorded there first, so a later copy into
// any of them waits for those readers (slot_rel_seq survives the clear).
int dsv4_slots_invalidate(dsv4_slots* s, void* compute_stream) {
  SREQ(s, DSV4_ERR_NULL, "slots: null handle");
  std::lock_guard<std::mutex> g(s->mu);
  SHIP(hipSetDevice(s->device));
  int rc = release_locked(s, (hipStream_t)compute_stream);
  if (rc) return rc;
  SHIP(hipStreamSynchronize(s->copy_stream));
  s->lru.clear();
  std::fill(s->slot_copy_seq.begin(), s->slot_copy_seq.end(), 0);
  return DSV4_OK;
}

// stats[0..8] = hits, misses, evictions, prefetched, bytes_h2d, copies, cached, capacity, pinned
int dsv4_slots_stats(dsv4_slots* s, int64_t* stats) {
  SREQ(s && stats, DSV4_ERR_NULL, "slots: null pointer");
  std::lock_guard<std::mutex> g(s->mu);
  stats[0] = s->hits;
  stats[1] = s->misses;
  stats[2] = s->evictions;
  stats[3] = s->prefetched;
  stats[4] = s->bytes_h2d;
  stats[5] = s->copies;
  stats[6] = s->lru.size();
  stats[7] = s->n_slots;
  stats[8] = s->pinned ? 1 : 0;
  return DSV4_OK;
}

int dsv4_slots_reset_stats(dsv4_slots* s) {
  SREQ(s, DSV4_ERR_NULL, "slots: null handle");
  std::lock_guard<std::mutex> g(s->mu);
  s->hits = s->misses = s->evictions = s->prefetched = s->bytes_h2d = s->copies = 0;
  return DSV4_OK;
}

}  // extern "C"
