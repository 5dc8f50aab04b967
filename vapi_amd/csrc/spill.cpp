// Spill tier: a host-memory store of exported KV blocks with an optional disk
// tier behind it, both least-recently-used (vapi's SpillStore,
// crates/vapi-cache/src/spill.rs:43-212), and the two engine steps that move
// blocks between it and the pool in batches (spill_evicted and the device
// half of promote_from_spill, crates/vapi-worker/src/engine.rs:369-456).
//
// Entries are keyed by the 32-byte block hash; a disk entry is the file
// "<64 lowercase hex>.kv" holding the block's blob in the export byte order
// (K of every layer, then V of every layer, each [block_size, kv_heads,
// head_dim]), so spill files are interchangeable with the reference's.
#include <hip/hip_runtime.h>

#include <sys/mman.h>

#include <cstdio>
#include <cstring>
#include <deque>
#include <filesystem>
#include <fstream>
#include <list>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "common.hpp"

using namespace vk;
namespace fs = std::filesystem;

namespace {

struct Hash {
  uint8_t b[32];
  bool operator==(const Hash& o) const { return std::memcmp(b, o.b, 32) == 0; }
};
struct HashHash {
  size_t operator()(const Hash& h) const {
    size_t x;
    std::memcpy(&x, h.b, sizeof(x));  // already a cryptographic hash
    return x;
  }
};

Hash to_hash(const uint8_t* p) {
  Hash h;
  std::memcpy(h.b, p, 32);
  return h;
}

std::string to_hex(const Hash& h) {
  static const char* d = "0123456789abcdef";
  std::string s(64, '0');
  for (int i = 0; i < 32; ++i) {
    s[2 * i] = d[h.b[i] >> 4];
    s[2 * i + 1] = d[h.b[i] & 15];
  }
  return s;
}

// Inverse of to_hex (either case, as from_str_radix accepts); false for any
// other name, so stray files in the directory are ignored.
bool from_hex(const std::string& s, Hash& h) {
  if (s.size() != 64) return false;
  auto nib = [](char c) -> int {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  };
  for (int i = 0; i < 32; ++i) {
    const int hi = nib(s[2 * i]), lo = nib(s[2 * i + 1]);
    if (hi < 0 || lo < 0) return false;
    h.b[i] = (uint8_t)(hi << 4 | lo);
  }
  return true;
}

// An LRU index: least recently used at the front.
template <typename V>
struct Lru {
  std::list<Hash> order;
  std::unordered_map<Hash, std::pair<V, std::list<Hash>::iterator>, HashHash> map;
  bool contains(const Hash& h) const { return map.count(h) != 0; }
  void push(const Hash& h, V v) {
    order.push_back(h);
    map.emplace(h, std::make_pair(std::move(v), std::prev(order.end())));
  }
  void touch(const Hash& h) {
    auto it = map.find(h);
    order.splice(order.end(), order, it->second.second);
  }
  V* find(const Hash& h) {
    auto it = map.find(h);
    return it == map.end() ? nullptr : &it->second.first;
  }
  bool pop_front(Hash& h, V& v) {
    if (order.empty()) return false;
    h = order.front();
    order.pop_front();
    auto it = map.find(h);
    v = std::move(it->second.first);
    map.erase(it);
    return true;
  }
  bool erase(const Hash& h, V& v) {
    auto it = map.find(h);
    if (it == map.end()) return false;
    v = std::move(it->second.first);
    order.erase(it->second.second);
    map.erase(it);
    return true;
  }
};

// Blob memory. A fresh 0.9 MB blob in ordinary heap memory takes a page
// fault per 4 KiB on first touch (~220 per block), which cost more than the
// copy itself; blobs of at least kArenaMin bytes are carved instead from
// 64 MiB chunks aligned to 2 MiB with transparent huge pages asked for
// (madvise), so a chunk faults in 2 MiB at a time. A freed blob goes to a
// free list of its size and is reused by the next blob of that size;
// chunks stay mapped until the process ends, but past kKeepFree bytes of
// free blobs (a store closed, or shrunk) a freed blob's pages are given back
// to the system (MADV_DONTNEED: its next use faults them in again).
class BlobArena {
 public:
  static constexpr size_t kArenaMin = 256 << 10;
  static constexpr size_t kChunk = 64ull << 20;
  static constexpr size_t kHuge = 2ull << 20;
  static constexpr size_t kKeepFree = 1ull << 30;

  static BlobArena& get() {
    static BlobArena* a = new BlobArena();  // never destroyed: blobs may outlive statics
    return *a;
  }
  void* allocate(size_t n) {
    const size_t sz = round_up(n, 4096);
    std::lock_guard<std::mutex> lk(mu_);
    auto it = free_.find(sz);
    if (it != free_.end() && !it->second.empty()) {
      void* p = it->second.back();
      it->second.pop_back();
      free_bytes_ -= sz;
      return p;
    }
    if (left_ < sz) {
      const size_t want = std::max(kChunk, round_up(sz, kHuge));
      // Over-map by one huge page and align the start to it.
      void* m = mmap(nullptr, want + kHuge, PROT_READ | PROT_WRITE,
                     MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
      if (m == MAP_FAILED) throw std::bad_alloc();
      char* base = (char*)round_up((size_t)(uintptr_t)m, kHuge);
      (void)madvise(base, want, MADV_HUGEPAGE);
      cur_ = base;
      left_ = want;
    }
    void* p = cur_;
    cur_ += sz;
    left_ -= sz;
    return p;
  }
  void deallocate(void* p, size_t n) {
    const size_t sz = round_up(n, 4096);
    std::lock_guard<std::mutex> lk(mu_);
    if (free_bytes_ + sz > kKeepFree) (void)madvise(p, sz, MADV_DONTNEED);
    free_[sz].push_back(p);
    free_bytes_ += sz;
  }

 private:
  static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
  std::mutex mu_;
  std::unordered_map<size_t, std::vector<void*>> free_;
  char* cur_ = nullptr;
  size_t left_ = 0;
  size_t free_bytes_ = 0;
};

template <typename T>
struct BlobAlloc {
  using value_type = T;
  BlobAlloc() = default;
  template <typename U>
  BlobAlloc(const BlobAlloc<U>&) {}
  T* allocate(size_t n) {
    const size_t bytes = n * sizeof(T);
    if (bytes < BlobArena::kArenaMin) return (T*)::operator new(bytes);
    return (T*)BlobArena::get().allocate(bytes);
  }
  void deallocate(T* p, size_t n) {
    const size_t bytes = n * sizeof(T);
    if (bytes < BlobArena::kArenaMin) ::operator delete(p);
    else BlobArena::get().deallocate(p, bytes);
  }
  template <typename U>
  bool operator==(const BlobAlloc<U>&) const { return true; }
  template <typename U>
  bool operator!=(const BlobAlloc<U>&) const { return false; }
};

// A stored blob's bytes.
using Bytes = std::vector<uint8_t, BlobAlloc<uint8_t>>;

// f(i) for i in [0, n) on up to 8 threads: the blob copies of a batch
// (page faults of fresh host memory and the copy itself) cost ~150 us per
// 0.9 MB block on one thread, several times the PCIe transfer.
template <typename F>
void parallel_for(uint32_t n, F f) {
  const uint32_t t = std::min<uint32_t>(n, std::max(1u, std::min(8u, std::thread::hardware_concurrency())));
  if (t <= 1) {
    for (uint32_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::vector<std::thread> pool;
  for (uint32_t k = 0; k < t; ++k)
    pool.emplace_back([&, k] {
      for (uint32_t i = k; i < n; i += t) f(i);
    });
  for (auto& th : pool) th.join();
}

}  // namespace

// Block ids from the host must name blocks of the pool (the kernels would
// otherwise skip them silently).
static int check_ids(const vapi_kv_pool* pool, const uint32_t* ids, uint32_t n, const char* who) {
  for (uint32_t i = 0; i < n; ++i)
    if (ids[i] >= pool->num_blocks)
      VK_FAIL(VAPI_KV_EINVAL, "%s: block %u of %u", who, ids[i], pool->num_blocks);
  return 0;
}

constexpr size_t kMaxInflight = 16;  // asynchronous exports in flight per store

struct vapi_spill_store {
  Lru<Bytes> ram;
  uint64_t ram_max = 0, ram_bytes = 0;
  bool has_dir = false;
  fs::path dir;
  Lru<uint64_t> disk;  // value: file length
  uint64_t disk_max = 0, disk_bytes = 0;
  vapi_spill_stats st{};

  // Asynchronous exports in flight, oldest first: the blobs of `hashes`,
  // back to back at `blobs` (pinned) once `copied` has completed. Each owns
  // the caller's staging and pinned ranges until it is drained. Events are
  // created on first use (a store without a GPU never needs them) and
  // recycled.
  struct Inflight {
    std::vector<Hash> hashes;
    const uint8_t* blobs;
    size_t bb;
    uintptr_t pin_lo, pin_hi, stg_lo, stg_hi;
    hipEvent_t packed, copied;
  };
  std::deque<Inflight> inflight;
  std::unordered_map<Hash, uint32_t, HashHash> in_flight_hashes;  // hash -> count
  std::vector<hipEvent_t> spare_events;

  ~vapi_spill_store() {
    for (auto& e : inflight) (void)hipEventSynchronize(e.copied);
    for (auto& e : inflight) spare_events.push_back(e.packed), spare_events.push_back(e.copied);
    for (hipEvent_t e : spare_events) (void)hipEventDestroy(e);
  }

  fs::path path(const Hash& h) const { return dir / (to_hex(h) + ".kv"); }

  void evict_disk() {
    Hash h;
    uint64_t len;
    while (disk_bytes > disk_max && disk.pop_front(h, len)) {
      std::error_code ec;
      fs::remove(path(h), ec);
      disk_bytes -= len;
    }
  }

  // Buffers of entries that left host memory, kept for the next copies in
  // (a fresh buffer costs a page fault per 4 KiB on first touch; a full
  // store recycles its evictions instead). Bounded by kSpareMax bytes and
  // by the host-memory cap.
  static constexpr uint64_t kSpareMax = 256ull << 20;
  std::vector<Bytes> spare;
  uint64_t spare_bytes = 0;

  void recycle(Bytes&& b) {
    if (spare_bytes + b.capacity() > std::min(kSpareMax, ram_max)) return;
    spare_bytes += b.capacity();
    spare.push_back(std::move(b));
  }

  // `n` buffers of `len` bytes (contents undefined): recycled ones first.
  std::vector<Bytes> buffers(uint32_t n, size_t len) {
    std::vector<Bytes> out(n);
    for (uint32_t j = 0; j < n && !spare.empty(); ++j) {
      if (spare.back().capacity() < len) break;
      spare_bytes -= spare.back().capacity();
      out[j] = std::move(spare.back());
      spare.pop_back();
      out[j].resize(len);
    }
    return out;
  }

  // Push host-memory entries out to disk until the cap is met.
  void evict_ram() {
    Hash h;
    Bytes bytes;
    while (ram_bytes > ram_max && ram.pop_front(h, bytes)) {
      ram_bytes -= bytes.size();
      if (!has_dir || bytes.size() > disk_max) {
        ++st.drops;
        recycle(std::move(bytes));
        continue;
      }
      std::ofstream f(path(h), std::ios::binary | std::ios::trunc);
      f.write((const char*)bytes.data(), (std::streamsize)bytes.size());
      f.close();
      if (!f) {
        ++st.errors;
        continue;
      }
      disk_bytes += bytes.size();
      disk.push(h, bytes.size());
      evict_disk();
      recycle(std::move(bytes));
    }
  }

  bool holds(const Hash& h) const { return ram.contains(h) || disk.contains(h); }

  // SpillStore::put (spill.rs:128-146), taking the blob's buffer.
  void put(const Hash& h, Bytes&& bytes) {
    if (holds(h)) return;
    const uint64_t len = bytes.size();
    if (len > ram_max && len > disk_max) {
      ++st.drops;
      return;
    }
    ++st.writes;
    ram_bytes += len;
    ram.push(h, std::move(bytes));
    evict_ram();
  }
  void put(const Hash& h, const uint8_t* p, size_t len) {
    if (holds(h)) return;
    put(h, Bytes(p, p + len));
  }

  // The entry's bytes into `out` (capacity `cap`): its length, -1 if not
  // held, VAPI_KV_ESPACE (nothing counted) if it does not fit.
  int64_t get(const Hash& h, void* out, size_t cap) {
    if (auto* v = ram.find(h)) {
      if (v->size() > cap) return VAPI_KV_ESPACE;
      std::memcpy(out, v->data(), v->size());
      ram.touch(h);
      ++st.hits;
      return (int64_t)v->size();
    }
    if (auto* len = disk.find(h)) {
      if (*len > cap) return VAPI_KV_ESPACE;
      std::ifstream f(path(h), std::ios::binary);
      const uint64_t n = *len;
      if (f && f.read((char*)out, (std::streamsize)n) && f.gcount() == (std::streamsize)n) {
        disk.touch(h);
        ++st.hits;
        return (int64_t)n;
      }
      uint64_t gone;  // deleted under us, or unreadable: forget it
      disk.erase(h, gone);
      disk_bytes -= gone;
      ++st.errors;
    }
    ++st.misses;
    return -1;
  }

  // Puts the blobs of in-flight exports into the store, oldest first: the
  // first `force` of them after waiting for their copies, then the rest
  // while their copies have completed (all of them if `wait`). Returns the
  // blobs stored or a negative error.
  int64_t drain(bool wait, size_t force = 0) {
    int64_t stored = 0;
    while (!inflight.empty()) {
      Inflight& e = inflight.front();
      if (wait || force) {
        VK_HIP(hipEventSynchronize(e.copied));
      } else {
        const hipError_t q = hipEventQuery(e.copied);
        if (q == hipErrorNotReady) break;
        if (q != hipSuccess) VK_FAIL(VAPI_KV_EHIP, "vapi_spill_drain: %s", hipGetErrorString(q));
      }
      if (force) --force;
      const uint32_t m = (uint32_t)e.hashes.size();
      std::vector<Bytes> copies = buffers(m, e.bb);
      parallel_for(m, [&](uint32_t j) {
        if (copies[j].size() == e.bb) std::memcpy(copies[j].data(), e.blobs + (size_t)j * e.bb, e.bb);
        else copies[j].assign(e.blobs + (size_t)j * e.bb, e.blobs + (size_t)(j + 1) * e.bb);
      });
      for (uint32_t j = 0; j < m; ++j) {
        put(e.hashes[j], std::move(copies[j]));
        auto it = in_flight_hashes.find(e.hashes[j]);
        if (it != in_flight_hashes.end() && --it->second == 0) in_flight_hashes.erase(it);
      }
      spare_events.push_back(e.packed);
      spare_events.push_back(e.copied);
      inflight.pop_front();
      stored += m;
    }
    return stored;
  }

  // Drains (waiting) every in-flight export up to the newest one whose
  // buffers overlap [pin_lo, pin_hi) or [stg_lo, stg_hi).
  int64_t release(uintptr_t pin_lo, uintptr_t pin_hi, uintptr_t stg_lo, uintptr_t stg_hi) {
    size_t upto = 0;
    for (size_t i = 0; i < inflight.size(); ++i) {
      const Inflight& e = inflight[i];
      const bool hit = (e.pin_lo < pin_hi && pin_lo < e.pin_hi) ||
                       (e.stg_lo < stg_hi && stg_lo < e.stg_hi) ||
                       (e.pin_lo < stg_hi && stg_lo < e.pin_hi) ||
                       (e.stg_lo < pin_hi && pin_lo < e.stg_hi);
      if (hit) upto = i + 1;
    }
    return upto ? drain(false, upto) : 0;
  }

  hipEvent_t event() {
    if (!spare_events.empty()) {
      hipEvent_t e = spare_events.back();
      spare_events.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
    return e;
  }
};

extern "C" {

int vapi_spill_open(const char* dir, uint64_t ram_max, uint64_t disk_max,
                    vapi_spill_store** out) {
  clear_error();
  if (!out) VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_open: null out");
  *out = nullptr;
  auto* s = new vapi_spill_store();
  s->ram_max = ram_max;
  s->disk_max = disk_max;
  if (dir && *dir && disk_max > 0) {
    std::error_code ec;
    fs::create_directories(dir, ec);
    if (ec) {
      delete s;
      VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_open: cannot create %s: %s", dir,
              ec.message().c_str());
    }
    s->dir = dir;
    s->has_dir = true;
    // Index what a previous run left: a hash pins the model and its
    // weights, so those blocks are still valid.
    for (const auto& e : fs::directory_iterator(s->dir, ec)) {
      Hash h;
      if (!e.is_regular_file() || e.path().extension() != ".kv" ||
          !from_hex(e.path().stem().string(), h))
        continue;
      const uint64_t len = e.file_size();
      s->disk.push(h, len);
      s->disk_bytes += len;
    }
    s->evict_disk();
  }
  *out = s;
  return 0;
}

void vapi_spill_close(vapi_spill_store* s) { delete s; }

int vapi_spill_contains(const vapi_spill_store* s, const uint8_t* hash) {
  if (!s || !hash) return 0;
  const Hash h = to_hash(hash);
  return s->ram.contains(h) || s->disk.contains(h);
}

int vapi_spill_put(vapi_spill_store* s, const uint8_t* hash, const void* bytes, size_t len) {
  clear_error();
  if (!s || !hash || (len && !bytes)) VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_put: null argument");
  if (int64_t rc = s->drain(false); rc < 0) return (int)rc;
  s->put(to_hash(hash), (const uint8_t*)bytes, len);
  return 0;
}

int64_t vapi_spill_get(vapi_spill_store* s, const uint8_t* hash, void* out, size_t cap) {
  clear_error();
  if (!s || !hash || (cap && !out)) VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_get: null argument");
  // A blob still in flight is waited for; completed exports enter anyway.
  if (int64_t rc = s->drain(s->in_flight_hashes.count(to_hash(hash)) > 0); rc < 0) return rc;
  const int64_t n = s->get(to_hash(hash), out, cap);
  if (n == VAPI_KV_ESPACE) VK_FAIL(VAPI_KV_ESPACE, "vapi_spill_get: %zu bytes is too small", cap);
  return n;
}

void vapi_spill_get_stats(const vapi_spill_store* s, vapi_spill_stats* out) {
  if (!s || !out) return;
  *out = s->st;
  out->ram_blocks = s->ram.map.size();
  out->ram_bytes = s->ram_bytes;
  out->disk_blocks = s->disk.map.size();
  out->disk_bytes = s->disk_bytes;
}

// spill_evicted (engine.rs:369-393) for n evicted blocks at once: the blocks
// the store does not hold yet are exported with vapi_kv_export_blocks into
// `pinned` (hipHostMalloc memory the kernel writes directly; the block ids
// are staged at its start) in as many rounds as it needs, and each blob is
// put into the store; with room for two blocks the buffer is used in two
// halves, so one round's export overlaps the previous round's copies.
// Returns the number exported; the blocks may be overwritten once it
// returns.
int64_t vapi_spill_evicted(vapi_spill_store* s, const vapi_kv_pool* pool, const uint32_t* ids,
                           const uint8_t* hashes, uint32_t n, void* pinned, size_t pinned_bytes,
                           vapi_stream_t stream) {
  clear_error();
  if (int rc = check_pool(pool, "vapi_spill_evicted")) return rc;
  if (!s || (n && (!ids || !hashes || !pinned)))
    VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_evicted: null argument");
  if (int rc = check_ids(pool, ids, n, "vapi_spill_evicted")) return rc;
  if (int64_t rc = s->drain(true); rc < 0) return rc;
  const size_t bb = vapi_kv_block_bytes(pool);
  const size_t head = 4096;  // id staging, 1,024 ids per round at most
  if (pinned_bytes < head + bb)
    VK_FAIL(VAPI_KV_ESPACE, "vapi_spill_evicted: %zu pinned bytes < %zu (one block)",
            pinned_bytes, head + bb);
  std::vector<uint32_t> todo;
  for (uint32_t i = 0; i < n; ++i)
    if (!vapi_spill_contains(s, hashes + 32ull * i)) todo.push_back(i);
  if (todo.empty()) return 0;
  // Two halves of the pinned buffer when it holds two blocks: the export
  // of round r + 1 runs on the GPU while round r is copied into the store.
  const size_t room = (pinned_bytes - head) / bb;
  const uint32_t halves = room >= 2 ? 2 : 1;
  const uint32_t per = (uint32_t)std::min<size_t>(room / halves, head / 4 / halves);
  const hipStream_t st = hs(stream);
  hipEvent_t ev[2] = {s->event(), halves == 2 ? s->event() : nullptr};
  auto give_back = [&] {
    for (hipEvent_t e : ev)
      if (e) s->spare_events.push_back(e);
  };
  if (!ev[0] || (halves == 2 && !ev[1])) {
    give_back();
    VK_FAIL(VAPI_KV_EHIP, "vapi_spill_evicted: hipEventCreate failed");
  }
  auto stage_ids = [&](uint32_t half) { return (uint32_t*)pinned + half * (head / 4 / halves); };
  auto stage_blobs = [&](uint32_t half) {
    return (uint8_t*)pinned + head + (size_t)half * per * bb;
  };
  const size_t rounds = (todo.size() + per - 1) / per;
  auto issue = [&](size_t r) -> int {
    const uint32_t half = (uint32_t)(r % halves);
    const size_t at = r * per;
    const uint32_t m = (uint32_t)std::min<size_t>(per, todo.size() - at);
    uint32_t* id_stage = stage_ids(half);
    for (uint32_t j = 0; j < m; ++j) id_stage[j] = ids[todo[at + j]];
    if (int rc = vapi_kv_export_blocks(pool, id_stage, m, stage_blobs(half), stream)) return rc;
    const hipError_t e = hipEventRecord(ev[half], st);
    if (e != hipSuccess) {
      set_error("vapi_spill_evicted: %s", hipGetErrorString(e));
      return VAPI_KV_EHIP;
    }
    return 0;
  };
  if (int rc = issue(0)) {
    give_back();
    return rc;
  }
  for (size_t r = 0; r < rounds; ++r) {
    const uint32_t half = (uint32_t)(r % halves);
    // Round r + 1 goes to the other half, whose previous round was copied
    // out before this iteration began.
    if (halves == 2 && r + 1 < rounds)
      if (int rc = issue(r + 1)) {
        (void)hipStreamSynchronize(st);
        give_back();
        return rc;
      }
    const hipError_t e = hipEventSynchronize(ev[half]);
    if (e != hipSuccess) {
      (void)hipStreamSynchronize(st);
      give_back();
      VK_FAIL(VAPI_KV_EHIP, "vapi_spill_evicted: %s", hipGetErrorString(e));
    }
    const size_t at = r * per;
    const uint32_t m = (uint32_t)std::min<size_t>(per, todo.size() - at);
    const uint8_t* blobs = stage_blobs(half);
    std::vector<Bytes> copies = s->buffers(m, bb);
    parallel_for(m, [&](uint32_t j) {
      if (copies[j].size() == bb) std::memcpy(copies[j].data(), blobs + (size_t)j * bb, bb);
      else copies[j].assign(blobs + (size_t)j * bb, blobs + (size_t)(j + 1) * bb);
    });
    for (uint32_t j = 0; j < m; ++j)
      s->put(to_hash(hashes + 32ull * todo[at + j]), std::move(copies[j]));
    if (halves == 1 && r + 1 < rounds)
      if (int rc = issue(r + 1)) {
        give_back();
        return rc;
      }
  }
  give_back();
  return (int64_t)todo.size();
}

// spill_evicted overlapped with the forward: the blocks the store neither
// holds nor has in flight are packed by vapi_kv_export_blocks into device
// staging on `stream` (an HBM-to-HBM copy; the forward may overwrite the
// blocks once it has run), then copied to `pinned` on `side`; a drain puts
// them into the store. Up to kMaxInflight exports are in flight, each on
// its own staging and pinned buffers (a ring the caller rotates); a call
// whose buffers overlap an in-flight export's first drains up to that one.
// staging and pinned (after its 4 KiB id stage) must hold every block to
// export, at most 1,024. Returns the number exported.
int64_t vapi_spill_evicted_async(vapi_spill_store* s, const vapi_kv_pool* pool,
                                 const uint32_t* ids, const uint8_t* hashes, uint32_t n,
                                 void* staging, size_t staging_bytes, void* pinned,
                                 size_t pinned_bytes, vapi_stream_t stream, vapi_stream_t side) {
  clear_error();
  if (int rc = check_pool(pool, "vapi_spill_evicted_async")) return rc;
  if (!s || (n && (!ids || !hashes || !pinned || !staging)))
    VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_evicted_async: null argument");
  if (int rc = check_ids(pool, ids, n, "vapi_spill_evicted_async")) return rc;
  const size_t bb = vapi_kv_block_bytes(pool);
  const size_t head = 4096;
  // Exports whose copies have completed enter the store now; the ones using
  // this call's buffers are waited for.
  if (int64_t rc = s->drain(false); rc < 0) return rc;
  const uintptr_t pin0 = (uintptr_t)pinned, stg0 = (uintptr_t)staging;
  if (int64_t rc = s->release(pin0, pin0 + pinned_bytes, stg0, stg0 + staging_bytes); rc < 0)
    return rc;
  if (s->inflight.size() >= kMaxInflight)
    if (int64_t rc = s->drain(false, s->inflight.size() - kMaxInflight + 1); rc < 0) return rc;
  std::vector<uint32_t> todo;
  for (uint32_t i = 0; i < n; ++i) {
    const Hash h = to_hash(hashes + 32ull * i);
    if (!s->holds(h) && !s->in_flight_hashes.count(h)) todo.push_back(i);
  }
  const uint32_t m = (uint32_t)todo.size();
  if (!m) return 0;
  if (m > head / 4 || staging_bytes < (size_t)m * bb || pinned_bytes < head + (size_t)m * bb)
    VK_FAIL(VAPI_KV_ESPACE,
            "vapi_spill_evicted_async: %u blocks of %zu bytes need %zu staging and %zu pinned "
            "bytes (at most 1024 blocks)",
            m, bb, (size_t)m * bb, head + (size_t)m * bb);
  vapi_spill_store::Inflight e;
  e.packed = s->event();
  e.copied = s->event();
  if (!e.packed || !e.copied) {
    if (e.packed) s->spare_events.push_back(e.packed);
    if (e.copied) s->spare_events.push_back(e.copied);
    VK_FAIL(VAPI_KV_EHIP, "vapi_spill_evicted_async: hipEventCreate failed");
  }
  uint32_t* id_stage = (uint32_t*)pinned;
  uint8_t* blobs = (uint8_t*)pinned + head;
  for (uint32_t j = 0; j < m; ++j) id_stage[j] = ids[todo[j]];
  auto fail = [&](int rc) {
    s->spare_events.push_back(e.packed);
    s->spare_events.push_back(e.copied);
    return rc;
  };
  if (int rc = vapi_kv_export_blocks(pool, id_stage, m, staging, stream)) return fail(rc);
  hipError_t err = hipEventRecord(e.packed, hs(stream));
  if (err == hipSuccess) err = hipStreamWaitEvent(hs(side), e.packed, 0);
  if (err == hipSuccess)
    err = hipMemcpyAsync(blobs, staging, (size_t)m * bb, hipMemcpyDeviceToHost, hs(side));
  if (err == hipSuccess) err = hipEventRecord(e.copied, hs(side));
  if (err != hipSuccess) {
    set_error("vapi_spill_evicted_async: %s", hipGetErrorString(err));
    return fail(VAPI_KV_EHIP);
  }
  e.blobs = blobs;
  e.bb = bb;
  e.pin_lo = pin0, e.pin_hi = pin0 + head + (size_t)m * bb;
  e.stg_lo = stg0, e.stg_hi = stg0 + (size_t)m * bb;
  e.hashes.reserve(m);
  for (uint32_t j = 0; j < m; ++j) {
    e.hashes.push_back(to_hash(hashes + 32ull * todo[j]));
    ++s->in_flight_hashes[e.hashes.back()];
  }
  s->inflight.push_back(std::move(e));
  return m;
}

int64_t vapi_spill_drain(vapi_spill_store* s, int wait) {
  clear_error();
  if (!s) VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_drain: null store");
  return s->drain(wait != 0);
}

// The device half of promote_from_spill (engine.rs:400-456): hashes[0..n)
// are a prompt's block chain and ids[0..n) the blocks allocated for them.
// Blobs are taken from the store in order up to the first it does not hold
// (only a contiguous prefix is worth restoring) and imported with
// vapi_kv_import_blocks through `pinned` (in two halves when it holds two
// blocks, so one round's copies overlap the previous round's import). A blob whose length is not
// vapi_kv_block_bytes is an error (backend.rs:739-745). Returns the number
// restored.
int64_t vapi_spill_promote(vapi_spill_store* s, const vapi_kv_pool* pool, const uint8_t* hashes,
                           const uint32_t* ids, uint32_t n, void* pinned, size_t pinned_bytes,
                           vapi_stream_t stream) {
  clear_error();
  if (int rc = check_pool(pool, "vapi_spill_promote")) return rc;
  if (!s || (n && (!ids || !hashes || !pinned)))
    VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_promote: null argument");
  if (int rc = check_ids(pool, ids, n, "vapi_spill_promote")) return rc;
  if (int64_t rc = s->drain(true); rc < 0) return rc;
  const size_t bb = vapi_kv_block_bytes(pool);
  const size_t head = 4096;
  if (pinned_bytes < head + bb)
    VK_FAIL(VAPI_KV_ESPACE, "vapi_spill_promote: %zu pinned bytes < %zu (one block)",
            pinned_bytes, head + bb);
  // Two halves of the pinned buffer when it holds two blocks: round r is
  // copied into one half while the GPU imports round r - 1 from the other.
  const size_t room = (pinned_bytes - head) / bb;
  const uint32_t halves = room >= 2 ? 2 : 1;
  const uint32_t per = (uint32_t)std::min<size_t>(room / halves, head / 4 / halves);
  const hipStream_t st = hs(stream);
  hipEvent_t ev[2] = {s->event(), halves == 2 ? s->event() : nullptr};
  struct Events {  // handed back to the store on every return
    vapi_spill_store* s;
    hipEvent_t* ev;
    ~Events() {
      for (int i = 0; i < 2; ++i)
        if (ev[i]) s->spare_events.push_back(ev[i]);
    }
  } events_guard{s, ev};
  if (!ev[0] || (halves == 2 && !ev[1]))
    VK_FAIL(VAPI_KV_EHIP, "vapi_spill_promote: hipEventCreate failed");
  uint32_t done = 0, round = 0;
  bool more = true;
  while (more && done < n) {
    const uint32_t half = round % halves;
    uint32_t* id_stage = (uint32_t*)pinned + half * (head / 4 / halves);
    uint8_t* blobs = (uint8_t*)pinned + head + (size_t)half * per * bb;
    // This half's previous import must have read its blobs.
    if (round >= halves) {
      const hipError_t e = hipEventSynchronize(ev[half]);
      if (e != hipSuccess)
        VK_FAIL(VAPI_KV_EHIP, "vapi_spill_promote: %s", hipGetErrorString(e));
    }
    // Resolve this batch's chain entries in order, copy (or read from disk)
    // their blobs into the pinned slots on several threads, then account
    // in order as a get() per entry would: LRU touch and hit, or for an
    // unreadable disk entry forget it, count the error and the miss and end
    // the chain there. A hash the store does not hold ends it too (a miss).
    struct Src {
      Hash h;
      const Bytes* ram;  // else on disk
      bool ok;
    };
    std::vector<Src> src;
    bool absent = false;
    while (src.size() < per && done + src.size() < n) {
      const Hash h = to_hash(hashes + 32ull * (done + src.size()));
      const Bytes* r = s->ram.find(h);
      const uint64_t* d = r ? nullptr : s->disk.find(h);
      if (!r && !d) {
        absent = true;
        break;
      }
      const uint64_t len = r ? r->size() : *d;
      if (len != bb) {
        (void)hipStreamSynchronize(st);  // earlier rounds' imports finish first
        VK_FAIL(VAPI_KV_EINVAL, "vapi_spill_promote: blob of %llu bytes, blocks are %zu",
                (unsigned long long)len, bb);
      }
      src.push_back(Src{h, r, false});
    }
    parallel_for((uint32_t)src.size(), [&](uint32_t k) {
      uint8_t* dst = blobs + (size_t)k * bb;
      if (src[k].ram) {
        std::memcpy(dst, src[k].ram->data(), bb);
        src[k].ok = true;
      } else {
        std::ifstream f(s->path(src[k].h), std::ios::binary);
        src[k].ok = f && f.read((char*)dst, (std::streamsize)bb) &&
                    f.gcount() == (std::streamsize)bb;
      }
    });
    uint32_t m = 0;
    for (; m < src.size(); ++m) {
      const Hash& h = src[m].h;
      if (!src[m].ok) {  // deleted under us, or unreadable: forget it
        uint64_t gone;
        s->disk.erase(h, gone);
        s->disk_bytes -= gone;
        ++s->st.errors;
        ++s->st.misses;
        more = false;
        break;
      }
      if (src[m].ram) s->ram.touch(h);
      else s->disk.touch(h);
      ++s->st.hits;
      id_stage[m] = ids[done + m];
    }
    if (more && absent) {
      ++s->st.misses;
      more = false;
    }
    if (!m) break;
    if (int rc = vapi_kv_import_blocks(pool, id_stage, m, blobs, stream)) {
      (void)hipStreamSynchronize(st);
      return rc;
    }
    VK_HIP(hipEventRecord(ev[half], st));
    done += m;
    ++round;
  }
  VK_HIP(hipStreamSynchronize(st));
  return done;
}

}  // extern "C"
