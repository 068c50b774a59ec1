// mkv_block.hip — GPU-resident block manager for prefix caching: a page-hash
// table, refcounts, copy-on-write forks and LRU eviction (gfx950).
//
// Semantics (one request at a time, in op order): see mkv_bm_step in mkv.h.
// Eviction order must equal a sequential OrderedDict model, so requests are
// processed in order by a single 1024-thread workgroup and the parallelism is
// inside a request: every page hash of a request is probed at once, pins and
// refcount updates are one lane per page, and allocation / release positions
// come from wavefront ballots + popcount prefix ranks.
//
// State (one caller-owned device buffer, layout from bm_layout):
//   counters  free_top, ring head/tail, next stamp, #evictable, tombstones,
//             eviction-log length
//   table     open addressing, linear probing: key[C] u64, val[C] i32
//             (-1 empty, -2 tombstone, -3 being written, >= 0 page id);
//             rebuilt when tombstones exceed C/4
//   per page  ref[P], flag[P] (bit 0: cached), stamp[P], hash[P], slot[P]
//             (the table slot of a cached page's key, so eviction needs no probe)
//   free      stack free[P] (pop from the top, like PagedKVCache.alloc_pages)
//   LRU       ring of (page, stamp) entries with lazy deletion: an entry is
//             live iff its page is cached, unreferenced and still carries that
//             stamp, so a page re-released later simply gets a newer entry —
//             exactly OrderedDict's move-to-end; eviction takes live entries
//             from the head (popitem(last=False)). Compacted in place (ballot
//             ranks) when full.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int kBmThreads = 1024;
constexpr int kBmWaves = kBmThreads / 64;

enum Ctr { kFreeTop, kHead, kTail, kNextStamp, kEvictable, kTombs, kLogLen, kNumCtr = 16 };
enum Status { kStOk = 0, kStOom = 1, kStBad = 2, kStReleased = 3 };

constexpr int32_t kEmpty = -1, kTomb = -2, kBusy = -3;

struct BmLayout {
  int64_t C, Q;  // table and ring capacities (powers of two)
  int64_t off_ctr, off_key, off_val, off_ref, off_flag, off_stamp, off_free, off_hash, off_ring_pg,
      off_ring_st, off_slot, bytes;
};

__host__ __device__ inline int64_t next_pow2(int64_t x) {
  int64_t p = 1024;
  while (p < x) p <<= 1;
  return p;
}

__host__ __device__ inline BmLayout bm_layout(int32_t P) {
  BmLayout l;
  l.C = next_pow2(4 * (int64_t)P);
  l.Q = next_pow2(2 * (int64_t)P);
  int64_t o = 0;
  auto take = [&o](int64_t n) {
    const int64_t at = o;
    o += (n + 255) / 256 * 256;
    return at;
  };
  l.off_ctr = take(kNumCtr * 8);
  l.off_key = take(l.C * 8);
  l.off_val = take(l.C * 4);
  l.off_ref = take((int64_t)P * 4);
  l.off_flag = take((int64_t)P * 4);
  l.off_stamp = take((int64_t)P * 4);
  l.off_free = take((int64_t)P * 4);
  l.off_hash = take((int64_t)P * 8);
  l.off_ring_pg = take(l.Q * 4);
  l.off_ring_st = take(l.Q * 4);
  l.off_slot = take((int64_t)P * 4);
  l.bytes = o;
  return l;
}

struct BmState {
  int64_t* ctr;
  uint64_t* key;
  int32_t* val;
  int32_t* ref;
  int32_t* flag;
  uint32_t* stamp;
  int32_t* free_list;
  uint64_t* hash;
  int32_t* ring_pg;
  uint32_t* ring_st;
  int32_t* slot;  // table slot holding a cached page's key
  int64_t C, Q;
  int32_t P;
};

inline BmState bm_state(void* base, int32_t P) {
  const BmLayout l = bm_layout(P);
  uint8_t* b = static_cast<uint8_t*>(base);
  BmState s;
  s.ctr = reinterpret_cast<int64_t*>(b + l.off_ctr);
  s.key = reinterpret_cast<uint64_t*>(b + l.off_key);
  s.val = reinterpret_cast<int32_t*>(b + l.off_val);
  s.ref = reinterpret_cast<int32_t*>(b + l.off_ref);
  s.flag = reinterpret_cast<int32_t*>(b + l.off_flag);
  s.stamp = reinterpret_cast<uint32_t*>(b + l.off_stamp);
  s.free_list = reinterpret_cast<int32_t*>(b + l.off_free);
  s.hash = reinterpret_cast<uint64_t*>(b + l.off_hash);
  s.ring_pg = reinterpret_cast<int32_t*>(b + l.off_ring_pg);
  s.ring_st = reinterpret_cast<uint32_t*>(b + l.off_ring_st);
  s.slot = reinterpret_cast<int32_t*>(b + l.off_slot);
  s.C = l.C;
  s.Q = l.Q;
  s.P = P;
  return s;
}

struct BmArgs {
  BmState s;
  const int32_t* ops;
  int32_t num_ops;
  int32_t num_requests;
  const uint64_t* hashes;
  const int64_t* hash_off;
  const int32_t* ntok;
  int32_t* tables;
  int64_t tstride;
  int32_t twidth;
  int32_t* hits;
  int32_t* child_last;
  int32_t* cow_src;
  int32_t* cow_dst;
  int32_t* status;
  int32_t* evict_log;
  int64_t evict_cap;
  int32_t* err;
};

// Per-workgroup scratch.
struct Shared {
  int32_t wave_sum[kBmWaves];
  int32_t first_miss;
  int32_t count;
  int32_t tomb_reused;
  int64_t new_head;
};

__device__ __forceinline__ uint32_t slot_of(uint64_t h) { return (uint32_t)(h ^ (h >> 29)); }

// Block-wide exclusive rank of a 0/1 flag (wavefront ballot + popcount, then
// the waves' totals through LDS). Every thread gets the block total. Contains
// barriers: every thread must call it.
__device__ __forceinline__ int32_t block_rank(bool flag, int32_t& total, Shared& sh) {
  const uint64_t m = __ballot(flag);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int32_t below = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) sh.wave_sum[wave] = __popcll(m);
  __syncthreads();
  int32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kBmWaves; ++w) {
    const int32_t c = sh.wave_sum[w];
    before += w < wave ? c : 0;
    all += c;
  }
  __syncthreads();
  total = all;
  return before + below;
}

// Page id under key h, or -1. Never runs concurrently with a writer of h.
__device__ int32_t tab_find(const BmState& s, uint64_t h, int64_t* slot_out = nullptr) {
  const int64_t mask = s.C - 1;
  int64_t i = slot_of(h) & mask;
  for (int64_t n = 0; n < s.C; ++n) {
    const int32_t v = __hip_atomic_load(&s.val[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (v == kEmpty) return -1;
    if (v >= 0 && s.key[i] == h) {
      if (slot_out) *slot_out = i;
      return v;
    }
    i = (i + 1) & mask;
  }
  return -1;
}

// Inserts h -> page (other lanes may insert other keys at the same time) and
// records the slot in slot[page]. Returns 1 if it reused a tombstone, 0 if it
// took an empty slot, -1 if the table was full (cannot happen: the load stays
// below 1/2 because of the rebuild threshold).
__device__ int32_t tab_insert(const BmState& s, uint64_t h, int32_t page) {
  const int64_t mask = s.C - 1;
  int64_t i = slot_of(h) & mask;
  for (int64_t n = 0; n < 2 * s.C; ++n) {
    const int32_t v = __hip_atomic_load(&s.val[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if ((v == kEmpty || v == kTomb) && atomicCAS(&s.val[i], v, kBusy) == v) {
      s.key[i] = h;
      s.slot[page] = (int32_t)i;
      __threadfence_block();
      __hip_atomic_store(&s.val[i], page, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      return v == kTomb ? 1 : 0;
    }
    if (v == kEmpty || v == kTomb) continue;  // lost the race for this slot: look again
    i = (i + 1) & mask;
  }
  return -1;
}

__device__ __forceinline__ bool ring_live(const BmState& s, int32_t pg, uint32_t st) {
  return (s.flag[pg] & 1) && s.ref[pg] == 0 && s.stamp[pg] == st;
}

// Counters every thread keeps in registers (all threads compute them alike).
struct Ctrs {
  int64_t free_top, head, tail, next_stamp, evictable, tombs, log_len;
};

// Moves the live ring entries [head, tail) to the front, in order.
__device__ void ring_compact(const BmArgs& a, Ctrs& c, Shared& sh) {
  const BmState& s = a.s;
  const int64_t qm = s.Q - 1;
  int64_t out = c.head;
  for (int64_t base = c.head; base < c.tail; base += kBmThreads) {
    const int64_t pos = base + threadIdx.x;
    bool live = false;
    int32_t pg = 0;
    uint32_t st = 0;
    if (pos < c.tail) {
      pg = s.ring_pg[pos & qm];
      st = s.ring_st[pos & qm];
      live = ring_live(s, pg, st);
    }
    int32_t total;
    const int32_t rank = block_rank(live, total, sh);  // all reads of this chunk are done
    if (live) {
      s.ring_pg[(out + rank) & qm] = pg;
      s.ring_st[(out + rank) & qm] = st;
    }
    out += total;
    __syncthreads();
  }
  c.tail = out;
}

// Rebuilds the hash table from the cached pages (drops every tombstone).
__device__ void tab_rebuild(const BmArgs& a, Ctrs& c) {
  const BmState& s = a.s;
  for (int64_t i = threadIdx.x; i < s.C; i += kBmThreads) s.val[i] = kEmpty;
  __syncthreads();
  for (int32_t p = threadIdx.x; p < s.P; p += kBmThreads)
    if (s.flag[p] & 1) tab_insert(s, s.hash[p], p);
  __syncthreads();
  c.tombs = 0;
}

// Probe results a thread keeps in registers for the pages it owns
// (i = tid + j*kBmThreads); requests longer than kHeld*kBmThreads pages re-read
// the rest from memory.
constexpr int kHeld = 4;

__device__ void admit(const BmArgs& a, int32_t r, Ctrs& c, Shared& sh) {
  const BmState& s = a.s;
  const int tid = threadIdx.x;
  const int32_t n = a.ntok[r];
  const int64_t h0 = a.hash_off[r];
  const int64_t m = a.hash_off[r + 1] - h0;
  const int64_t n_pages = (n + 15) / 16;
  const bool cow = (n & 15) != 0;
  int32_t* row = a.tables + (int64_t)r * a.tstride;
  if (n < 0 || m != n / 16 || n_pages > a.twidth) {
    if (tid == 0) {
      a.status[r] = kStBad;
      a.hits[r] = 0;
      a.child_last[r] = a.cow_src[r] = a.cow_dst[r] = -1;
      raise_err(a.err, MKV_DEVERR_BM);
    }
    return;
  }
  if (c.tombs > s.C / 4) tab_rebuild(a, c);

  // 1. probe every page hash; k = first miss. Each lane keeps the page and its
  //    current refcount for its first kHeld hashes.
  if (tid == 0) {
    sh.first_miss = (int32_t)m;
    sh.count = 0;
    sh.tomb_reused = 0;
  }
  __syncthreads();
  int32_t held_pg[kHeld], held_ref[kHeld];
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    held_pg[j] = -1;
    held_ref[j] = 0;
  }
  for (int64_t i = tid, j = 0; i < m; i += kBmThreads, ++j) {
    const int32_t p = tab_find(s, a.hashes[h0 + i]);
    row[i] = p;
    if (p < 0) atomicMin(&sh.first_miss, (int32_t)i);
    if (j < kHeld) {
      held_pg[j] = p;
      held_ref[j] = p >= 0 ? s.ref[p] : 0;
    }
  }
  __syncthreads();
  const int64_t k = sh.first_miss;

  // 2. hits that are evictable now will be pinned: count them for the OOM check
  {
    int32_t cnt = 0;
    for (int64_t i = tid, j = 0; i < k; i += kBmThreads, ++j)
      cnt += (j < kHeld ? held_ref[j] : s.ref[row[i]]) == 0;
    if (cnt) atomicAdd(&sh.count, cnt);
  }
  __syncthreads();
  const int64_t pinned = sh.count;
  const int64_t take = n_pages - k + (cow ? 1 : 0);
  if (take > c.free_top + c.evictable - pinned) {
    if (tid == 0) {
      a.status[r] = kStOom;
      a.hits[r] = 0;
      a.child_last[r] = a.cow_src[r] = a.cow_dst[r] = -1;
    }
    __syncthreads();
    return;
  }

  // 3. pin the hits, for the parent and the forked child at once (+2)
  for (int64_t i = tid, j = 0; i < k; i += kBmThreads, ++j) {
    if (j < kHeld)
      s.ref[held_pg[j]] = held_ref[j] + 2;
    else
      s.ref[row[i]] += 2;
  }
  c.evictable -= pinned;

  // 4. take pages: the free stack's top first, then LRU victims in order. The
  //    first n_pages-k go to the table (held by parent and child: refcount 2,
  //    except a partial last page, which the child copies: 1), the last (if
  //    any) is the child's copy (refcount 1).
  const int64_t from_free = take < c.free_top ? take : c.free_top;
  const int64_t table_new = n_pages - k;
  for (int64_t j = tid; j < from_free; j += kBmThreads) {
    const int32_t p = s.free_list[c.free_top - 1 - j];
    if (j < table_new) {
      row[k + j] = p;
      s.ref[p] = (cow && k + j == n_pages - 1) ? 1 : 2;
    } else {
      a.cow_dst[r] = p;
      s.ref[p] = 1;
    }
  }
  c.free_top -= from_free;
  int64_t done = from_free;
  const int64_t qm = s.Q - 1;
  while (done < take) {
    if (c.head >= c.tail) {  // fewer live entries than counted: state is corrupt
      if (tid == 0) raise_err(a.err, MKV_DEVERR_BM);
      break;
    }
    const int64_t pos = c.head + tid;
    bool live = false;
    int32_t pg = 0;
    if (pos < c.tail) {
      pg = s.ring_pg[pos & qm];
      live = ring_live(s, pg, s.ring_st[pos & qm]);
    }
    int32_t total;
    const int32_t rank = block_rank(live, total, sh);
    const int64_t want = take - done;
    if (live && rank < want) {
      const int64_t j = done + rank;
      s.val[s.slot[pg]] = kTomb;  // the page's key leaves the table
      s.flag[pg] &= ~1;
      if (j < table_new) {
        row[k + j] = pg;
        s.ref[pg] = (cow && k + j == n_pages - 1) ? 1 : 2;
      } else {
        a.cow_dst[r] = pg;
        s.ref[pg] = 1;
      }
      if (c.log_len + (j - from_free) < a.evict_cap)
        a.evict_log[c.log_len + (j - from_free)] = pg;
      if (rank == want - 1) sh.new_head = pos + 1;
    }
    __syncthreads();
    const int64_t got = total < want ? total : want;
    c.head = total >= want ? sh.new_head
                           : (c.head + kBmThreads < c.tail ? c.head + kBmThreads : c.tail);
    c.evictable -= got;
    c.tombs += got;
    done += got;
    __syncthreads();
  }
  c.log_len += done - from_free;

  // 5. register the new full pages' hashes unless already present. A key the
  //    probe did not find is still absent (only evictions ran since); a key
  //    it found is present unless its page was just evicted. All presence
  //    checks of a chunk finish before any of its inserts (barrier), so no
  //    check reads a page another lane is registering.
  for (int64_t base = 0; base < m; base += (int64_t)kHeld * kBmThreads) {
    bool reg[kHeld];
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
      const int64_t i = base + tid + (int64_t)j * kBmThreads;
      reg[j] = false;
      if (i < m && i >= k) {
        const uint64_t h = a.hashes[h0 + i];
        const int32_t seen = base == 0 ? held_pg[j] : tab_find(s, h);
        reg[j] = !(seen >= 0 && (s.flag[seen] & 1) && s.hash[seen] == h);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
      if (!reg[j]) continue;
      const int64_t i = base + tid + (int64_t)j * kBmThreads;
      const uint64_t h = a.hashes[h0 + i];
      const int32_t p = row[i];
      s.hash[p] = h;
      s.flag[p] |= 1;
      if (tab_insert(s, h, p) == 1) atomicAdd(&sh.tomb_reused, 1);
    }
    __syncthreads();
  }
  c.tombs -= sh.tomb_reused;

  if (tid == 0) {
    a.hits[r] = (int32_t)k;
    a.status[r] = kStOk;
    if (cow) {
      a.cow_src[r] = row[n_pages - 1];
      a.child_last[r] = a.cow_dst[r];
    } else {
      a.cow_src[r] = a.cow_dst[r] = -1;
      a.child_last[r] = n_pages ? row[n_pages - 1] : -1;
    }
  }
  __syncthreads();
}

// Releases a forked request in one pass. Sequentially that is the child's
// table then the parent's, each from its last page: refcount -= 1; at zero a
// cached page goes to the LRU's newest end, any other page onto the free
// stack. The child shares every page of the parent except, after a
// copy-on-write, the last (its own copy), so in one pass over the table from
// the last page: the child's copy (if any) reaches zero first and goes to the
// free stack; then every shared page loses both references at once, and the
// parent's own partial last page (after a copy) loses one. Pages reach zero
// in the same order as in the two sequential passes.
__device__ void release(const BmArgs& a, int32_t r, Ctrs& c, Shared& sh) {
  const BmState& s = a.s;
  const int32_t st = a.status[r];
  if (st != kStOk) {  // an OOM request holds nothing; anything else is a caller error
    if (st != kStOom && threadIdx.x == 0) raise_err(a.err, MKV_DEVERR_BM);
    return;
  }
  const int32_t n = a.ntok[r];
  const int64_t n_pages = (n + 15) / 16;
  const bool cow = (n & 15) != 0;
  const int32_t* row = a.tables + (int64_t)r * a.tstride;
  const int64_t qm = s.Q - 1;
  if (cow) {  // the child's private copy: uncached, refcount 1 -> free stack
    if (threadIdx.x == 0) {
      const int32_t p = a.child_last[r];
      s.ref[p] = 0;
      s.free_list[c.free_top] = p;
    }
    c.free_top += 1;
  }
  if (c.tail - c.head + n_pages > s.Q) ring_compact(a, c, sh);
  for (int64_t base = 0; base < n_pages; base += kBmThreads) {
    const int64_t j = base + threadIdx.x;  // j-th page from the tail
    bool to_lru = false, to_free = false;
    int32_t page = 0;
    if (j < n_pages) {
      const int64_t i = n_pages - 1 - j;
      page = row[i];
      const int32_t drop = (cow && i == n_pages - 1) ? 1 : 2;
      const int32_t left = s.ref[page] - drop;
      s.ref[page] = left;
      if (left == 0) {
        to_lru = (s.flag[page] & 1) != 0;
        to_free = !to_lru;
      }
    }
    int32_t n_lru, n_free;
    const int32_t rl = block_rank(to_lru, n_lru, sh);
    const int32_t rf = block_rank(to_free, n_free, sh);
    if (to_lru) {
      const uint32_t stamp = (uint32_t)(c.next_stamp + rl);
      s.ring_pg[(c.tail + rl) & qm] = page;
      s.ring_st[(c.tail + rl) & qm] = stamp;
      s.stamp[page] = stamp;
    }
    if (to_free) s.free_list[c.free_top + rf] = page;
    c.tail += n_lru;
    c.next_stamp += n_lru;
    c.evictable += n_lru;
    c.free_top += n_free;
    __syncthreads();
  }
  if (threadIdx.x == 0) a.status[r] = kStReleased;
  __syncthreads();
}

__global__ __launch_bounds__(kBmThreads) void bm_step_kernel(BmArgs a) {
  __shared__ Shared sh;
  Ctrs c;
  c.free_top = a.s.ctr[kFreeTop];
  c.head = a.s.ctr[kHead];
  c.tail = a.s.ctr[kTail];
  c.next_stamp = a.s.ctr[kNextStamp];
  c.evictable = a.s.ctr[kEvictable];
  c.tombs = a.s.ctr[kTombs];
  c.log_len = a.s.ctr[kLogLen];
  for (int32_t o = 0; o < a.num_ops; ++o) {
    const int32_t op = a.ops[o];
    const int32_t r = op >= 0 ? op : -(op + 1);
    if (r >= a.num_requests) {
      if (threadIdx.x == 0) raise_err(a.err, MKV_DEVERR_BM);
    } else if (op >= 0) {
      admit(a, r, c, sh);
    } else {
      release(a, r, c, sh);
    }
    __syncthreads();  // the op's writes are visible to the next op
  }
  if (threadIdx.x == 0) {
    a.s.ctr[kFreeTop] = c.free_top;
    a.s.ctr[kHead] = c.head;
    a.s.ctr[kTail] = c.tail;
    a.s.ctr[kNextStamp] = c.next_stamp;
    a.s.ctr[kEvictable] = c.evictable;
    a.s.ctr[kTombs] = c.tombs;
    a.s.ctr[kLogLen] = c.log_len;
  }
}

__global__ __launch_bounds__(256) void bm_init_kernel(BmState s, const int32_t* free_order) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = g; i < s.C; i += stride) s.val[i] = kEmpty;
  for (int64_t p = g; p < s.P; p += stride) {
    s.ref[p] = 0;
    s.flag[p] = 0;
    s.stamp[p] = 0;
    s.free_list[p] = free_order ? free_order[p] : (int32_t)p;
  }
  if (g < kNumCtr) s.ctr[g] = g == kFreeTop ? s.P : (g == kNextStamp ? 1 : 0);
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int64_t mkv_bm_state_bytes(int32_t num_pages) {
  if (num_pages <= 0 || num_pages > (1 << 28)) return -1;
  return bm_layout(num_pages).bytes;
}

extern "C" int mkv_bm_layout(int32_t num_pages, int64_t* out) {
  clear_error();
  MKV_REQUIRE(num_pages > 0 && num_pages <= (1 << 28) && out, MKV_E_INVALID,
              "mkv_bm_layout: bad arguments");
  const BmLayout l = bm_layout(num_pages);
  const int64_t v[14] = {l.C,        l.Q,        l.off_ctr,   l.off_key,     l.off_val,
                         l.off_ref,  l.off_flag, l.off_stamp, l.off_free,    l.off_hash,
                         l.off_ring_pg, l.off_ring_st, l.off_slot, l.bytes};
  for (int i = 0; i < 14; ++i) out[i] = v[i];
  return MKV_OK;
}

extern "C" int mkv_bm_init(void* state, int32_t num_pages, const int32_t* free_order,
                           void* stream) {
  clear_error();
  MKV_REQUIRE(state && num_pages > 0 && num_pages <= (1 << 28), MKV_E_INVALID,
              "mkv_bm_init: bad arguments");
  MKV_REQUIRE(((uintptr_t)state & 255) == 0, MKV_E_ALIGN,
              "mkv_bm_init: state must be 256-byte aligned");
  const BmState s = bm_state(state, num_pages);
  hipLaunchKernelGGL(bm_init_kernel, dim3(1024), dim3(256), 0, as_stream(stream), s, free_order);
  return check_launch("mkv_bm_init");
}

extern "C" int mkv_bm_step(void* state, int32_t num_pages, const int32_t* ops, int32_t num_ops,
                           int32_t num_requests, const uint64_t* page_hashes, const int64_t* hash_offsets,
                           const int32_t* num_tokens, int32_t* tables, int64_t table_stride,
                           int32_t table_width, int32_t* hits, int32_t* child_last,
                           int32_t* cow_src, int32_t* cow_dst, int32_t* status,
                           int32_t* evict_log, int64_t evict_log_capacity, int32_t* err,
                           void* stream) {
  clear_error();
  MKV_REQUIRE(num_ops >= 0 && num_pages > 0 && table_width >= 0 && num_requests >= 0,
              MKV_E_INVALID, "mkv_bm_step: bad sizes");
  if (num_ops == 0) return MKV_OK;
  MKV_REQUIRE(state && ops && hash_offsets && num_tokens && tables && hits && child_last &&
                  cow_src && cow_dst && status && err,
              MKV_E_INVALID, "mkv_bm_step: null pointer");
  MKV_REQUIRE(evict_log || evict_log_capacity == 0, MKV_E_INVALID,
              "mkv_bm_step: eviction log capacity without a log");
  BmArgs a;
  a.s = bm_state(state, num_pages);
  a.ops = ops;
  a.num_ops = num_ops;
  a.num_requests = num_requests;
  a.hashes = page_hashes;
  a.hash_off = hash_offsets;
  a.ntok = num_tokens;
  a.tables = tables;
  a.tstride = table_stride;
  a.twidth = table_width;
  a.hits = hits;
  a.child_last = child_last;
  a.cow_src = cow_src;
  a.cow_dst = cow_dst;
  a.status = status;
  a.evict_log = evict_log;
  a.evict_cap = evict_log_capacity;
  a.err = err;
  hipLaunchKernelGGL(bm_step_kernel, dim3(1), dim3(kBmThreads), 0, as_stream(stream), a);
  return check_launch("mkv_bm_step");
}
