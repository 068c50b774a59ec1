// mkv_block.hip — GPU-resident block manager for prefix caching: a page-hash
// table, refcounts, copy-on-write forks and LRU eviction (gfx950).
//
// Semantics (one request at a time, in op order): see mkv_bm_step in mkv.h.
// Eviction order must equal a sequential OrderedDict model, so requests are
// resolved in order by one 512-thread workgroup, and the parallelism is inside
// a request: every page hash of a request is probed at once, pins and
// refcount updates are one lane per page, and allocation / release positions
// come from wavefront ballots + popcount prefix ranks. A leading run of
// releases is retired on many CUs, and the admits after it are resolved
// speculatively on many CUs up to the first one the speculation cannot
// vouch for. The tail kernel takes the rest: admits eight at a time in its
// group pass (one round of loads for the eight, then a sequential resolution
// in LDS), then whatever is left one op at a time in its step pass. A step is
// ten launches: setup (one workgroup), drop, mark, push + probe, hits,
// window, victims, commit, finish, tail (one workgroup).
//
// A request costs a few dependent memory round trips, so the layout keeps
// that chain short:
//   * a table entry holds key, page id and (mirrored) the page's refcount in
//     16 bytes: one load per probe step answers "cached, and evictable?";
//   * a page's refcount, flags, LRU stamp and the table slot of its key are the
//     first 16 bytes of its 32-byte record: one load tells whether the page is
//     evictable and where its key lives;
//   * an LRU ring entry is one 8-byte (page, stamp) pair;
//   * the ops' request metadata is staged in LDS, the next request's page
//     hashes are loaded while the current request runs, and the free-stack
//     entries a request may take are loaded with its probe;
//   * the probe remembers where a missing key would go, so registering it is
//     a plain store (the slot claimed in LDS);
//   * the number of hits that leave the LRU comes from per-wave ballots kept
//     in LDS, without another reduction.
//
// State (one caller-owned device buffer, layout from bm_layout):
//   counters  free_top, ring head/tail, next stamp, #evictable, tombstones,
//             eviction-log length
//   table     ent[C] {u64 key, i32 page (-1 empty, -2 tombstone, -3 being
//             written), i32 the page's refcount (a copy of rec.ref, kept
//             equal while the page is cached)}: open addressing, linear
//             probing; rebuilt when tombstones exceed C/4
//   pages     rec[P] {i32 ref, i32 flag (bit 0: cached), u32 stamp, i32 table
//             slot of the page's key, u64 hash, u64 unused}
//   free      stack free[P] (pop from the top, like PagedKVCache.alloc_pages)
//   LRU       ring[Q] of page | stamp << 32 with lazy deletion: an entry is
//             live iff its page is cached, unreferenced and still carries that
//             stamp, so a page re-released later simply gets a newer entry —
//             exactly OrderedDict's move-to-end; eviction takes live entries
//             from the head (popitem(last=False)). Compacted in place (ballot
//             ranks) when full.
#include <climits>

#include "mkv_device.h"

namespace mkv {
namespace {

// 512 threads: a request's pages fit (up to 512 in registers), and every
// wave runs the per-request bookkeeping, so more waves cost more than they
// add (1024 and 256 threads measured slower).
constexpr int kBmThreads = 512;
constexpr int kBmWaves = kBmThreads / 64;
constexpr int kOpChunk = 1024;  // ops whose request metadata is staged in LDS at once
// Page hashes (and probe results) a thread keeps in registers: pages
// tid + j*kBmThreads for j < kHeld. Longer requests re-read the rest.
constexpr int kHeld = 1;
constexpr int kSetSize = 2048;  // LDS set of the table slots an admit claims
static_assert(kSetSize == 1 << 11, "set_add's default size");

enum Ctr { kFreeTop, kHead, kTail, kNextStamp, kEvictable, kTombs, kLogLen,
           kSpecDone,  // admits resolved by the speculation, since init
           kSpecLeft,  // admits it covered but left to the sequential path, since init
           kNumCtr = 16 };
enum Status { kStOk = 0, kStOom = 1, kStBad = 2, kStReleased = 3 };

constexpr int32_t kEmpty = -1, kTomb = -2, kBusy = -3;
constexpr int64_t kEntBytes = 16, kRecBytes = 32;

// A leading run of release ops is retired by multi-workgroup kernels before
// the one-workgroup tail kernel runs the rest (see the run kernels below); its
// scratch lives in the state buffer.
constexpr int kRunMaxOps = 1024;               // releases retired in bulk per step
constexpr int64_t kRunMaxElems = 1 << 20;      // their page references
// The run takes a single leading release too: the speculation starts after
// the run, so a release left to the tail kernel would leave every admit
// after it to the one-workgroup kernel.
constexpr int kRunMinOps = 1;
// A step of at most this many ops runs on the one-workgroup tail kernel alone:
// one launch, against ten dependent launches of a few microseconds each,
// which a concurrent kernel that fills the GPU stretches to tens each.
constexpr int kShortStepOps = 8;
constexpr int64_t kRunMaxWords = kRunMaxElems / 32;
// The run's elements (and the ring entries a compaction copies) are counted in
// chunks of kRunChunk: a workgroup of the mark pass writes each chunk's set
// bits per array and each bit word's count before it within the chunk, and a
// workgroup of the push pass adds up the chunks before its own.
constexpr int kRunChunk = 256;
constexpr int64_t kRunMaxChunks = kRunMaxElems / kRunChunk;
enum RunCtr { kRunOps, kRunTotal,
              kRunTail0, kRunStamp0, kRunFree0, kRunEvict0,  // counters before the run
              kRunCompact, kRunSpan,
              kRunNext,  // the first op left to the next stage (speculation, groups, step)
              kRunNumCtr = 16 };

// The speculative resolution of a step's admits (many CUs; see the
// speculation kernels): up to kSpecOps admits of up to kSpecPos pages each,
// a first-occurrence table of absent keys, and an LRU window of kSpecWin
// entries.
constexpr int kSpecOps = 1024;
constexpr int kSpecPos = 2048;
constexpr int kFoBits = 19;
constexpr int64_t kFoCap = 1ll << kFoBits;
constexpr int kFoMaxProbe = 512;  // a longer probe counts as a violation
constexpr int kSpecWin = 1 << 17;
constexpr int kWinChunk = 256;                     // window entries per candidate count
constexpr int kWinChunks = kSpecWin / kWinChunk;
enum SpecCtr { kSpN,        // admits speculated
               kSpBad,      // first admit the speculation may get wrong (<= kSpN)
               kSpF,        // free-stack entries at the step's start
               kSpLive,     // evictable pages at the step's start
               kSpHead,     // LRU head at the step's start
               kSpWin,      // window entries read
               kSpReused,   // registrations that reused a tombstone
               kSpNumCtr = 16 };

struct BmLayout {
  int64_t C, Q;  // table and ring capacities (powers of two)
  int64_t off_ctr, off_ent, off_rec, off_free, off_ring, off_last, off_run, bytes;
  // inside the run scratch at off_run
  int64_t run_ctr, run_off, run_child, run_page, run_bits, run_wpre, run_ccnt;
  // ring compaction scratch: a copy of the ring span, live bits, their counts
  int64_t cmp_ring, cmp_bits, cmp_pre, cmp_ccnt;
  // speculation scratch
  int64_t sp_ctr, sp_req, sp_ntok, sp_m, sp_h0, sp_k, sp_take, sp_pinned, sp_T, sp_p0, sp_fo,
      sp_first, sp_late, sp_wpg, sp_wslot, sp_wflag, sp_victim, sp_vpos, sp_wcnt;
};

__host__ __device__ inline int64_t next_pow2(int64_t x) {
  int64_t p = 1024;
  while (p < x) p <<= 1;
  return p;
}

__host__ __device__ inline BmLayout bm_layout(int32_t P) {
  BmLayout l;
  // 32 entries per page (at most 2^30, so slots stay int32; at least 4 per
  // page): an admit waits for the longest probe chain among its hundreds of
  // parallel lookups, so a sparse table pays (prefix trace: 22.9 ms of
  // manager time at 4 entries per page, 18.5 at 16, 18.0 at 32, 17.7 at 64)
  l.C = next_pow2(32 * (int64_t)P < (1LL << 30) ? 32 * (int64_t)P : (1LL << 30));
  l.Q = next_pow2(2 * (int64_t)P);
  int64_t o = 0;
  auto take = [&o](int64_t n) {
    const int64_t at = o;
    o += (n + 255) / 256 * 256;
    return at;
  };
  l.off_ctr = take(kNumCtr * 8);
  l.off_ent = take(l.C * kEntBytes);
  l.off_rec = take((int64_t)P * kRecBytes);
  l.off_free = take((int64_t)P * 4);
  l.off_ring = take(l.Q * 8);
  l.off_last = take((int64_t)P * 4);
  l.off_run = o;
  l.run_ctr = take(kRunNumCtr * 8);
  l.run_off = take((kRunMaxOps + 1) * 8);
  l.run_child = take(kRunMaxOps * 4);
  l.run_page = take(kRunMaxElems * 4);
  l.run_bits = take(3 * kRunMaxWords * 4);
  l.run_wpre = take(2 * kRunMaxWords * 4);
  l.run_ccnt = take(2 * kRunMaxChunks * 4);
  l.cmp_ring = take(l.Q * 8);
  l.cmp_bits = take(l.Q / 32 * 4);
  l.cmp_pre = take(l.Q / 32 * 4);
  l.cmp_ccnt = take(l.Q / kRunChunk * 4);
  l.sp_ctr = take(kSpNumCtr * 8);
  l.sp_req = take(kSpecOps * 4);
  l.sp_ntok = take(kSpecOps * 4);
  l.sp_m = take(kSpecOps * 4);
  l.sp_h0 = take(kSpecOps * 8);
  l.sp_k = take(kSpecOps * 4);
  l.sp_take = take(kSpecOps * 4);
  l.sp_pinned = take(kSpecOps * 4);
  l.sp_T = take((kSpecOps + 1) * 8);
  l.sp_p0 = take((int64_t)kSpecOps * kSpecPos * 8);
  l.sp_fo = take(kFoCap * 16);
  l.sp_first = take((int64_t)P * 4);
  l.sp_late = take((int64_t)P * 4);
  l.sp_wpg = take(kSpecWin * 4);
  l.sp_wslot = take(kSpecWin * 4);
  l.sp_wflag = take(kSpecWin);
  l.sp_victim = take(kSpecWin * 4);
  l.sp_vpos = take(kSpecWin * 4);
  l.sp_wcnt = take(kWinChunks * 4);
  l.bytes = o;
  return l;
}

struct BmState {
  int64_t* ctr;
  uint8_t* ent;  // C x 16 bytes
  uint8_t* rec;  // P x 32 bytes
  int32_t* free_list;
  uint64_t* ring;
  int32_t* last;       // run: a page's last position in the run (-1 between runs)
  int64_t* run_ctr;    // run: RunCtr values
  int64_t* run_off;    // run: element offset of each op of the run
  int32_t* run_child;  // run: the op's child copy page, -1 none, -2 releases nothing
  int32_t* run_page;   // run: page id of each element
  uint32_t* run_bits;  // run: [3][kRunMaxWords] to the ring / free stack / last occurrence
  uint32_t* run_wpre;  // run: [2][kRunMaxWords] the first two's counts before each word,
                       //  within its chunk
  uint32_t* run_ccnt;  // run: [2][kRunMaxChunks] their set bits per chunk
  uint64_t* cmp_ring;  // compaction: the ring span [head, tail) copied out
  uint32_t* cmp_bits;  // compaction: live bit per copied entry
  uint32_t* cmp_pre;   // compaction: live entries before each bit word, within its chunk
  uint32_t* cmp_ccnt;  // compaction: live entries per chunk
  // speculation (per admit j < kSpecOps, position i < kSpecPos)
  int64_t* sp_ctr;     // SpecCtr values
  int32_t* sp_req;     // request id
  int32_t* sp_ntok;    // tokens
  int32_t* sp_m;       // page hashes
  int64_t* sp_h0;      // first page hash
  int32_t* sp_k;       // hits
  int32_t* sp_take;    // pages taken
  int32_t* sp_pinned;  // pages it pins (refcount 0 before, first admit to hit them)
  int64_t* sp_T;       // takes before it (exclusive prefix sum)
  int2* sp_p0;         // [j][i] {page | kPinBit at the step's start, or -1, or -(c+2) for
                       //  a key first held at occurrence c = admit * kSpecPos + position
                       //  of an earlier admit; table slot | kTombBit}
  uint8_t* sp_fo;      // first-occurrence table: {u64 key, i32 first occurrence, i32 -}
  int32_t* sp_first;   // [P] first admit pinning the page (INT_MAX none)
  int32_t* sp_late;    // [P] first admit holding the page (found at S) past its first miss
  int32_t* sp_wpg;     // [w] LRU window: page
  int32_t* sp_wslot;   //     its key's table slot
  uint8_t* sp_wflag;   //     0 dead, 1 a victim candidate, 2 live but pinned in the step
  int32_t* sp_victim;  // [v] the v-th eviction's page
  int32_t* sp_vpos;    //     its window position
  int32_t* sp_wcnt;    // [c] victim candidates in window chunk c (kWinChunk entries)
  int64_t C, Q;
  int32_t P;
};

inline BmState bm_state(void* base, int32_t P) {
  const BmLayout l = bm_layout(P);
  uint8_t* b = static_cast<uint8_t*>(base);
  BmState s;
  s.ctr = reinterpret_cast<int64_t*>(b + l.off_ctr);
  s.ent = b + l.off_ent;
  s.rec = b + l.off_rec;
  s.free_list = reinterpret_cast<int32_t*>(b + l.off_free);
  s.ring = reinterpret_cast<uint64_t*>(b + l.off_ring);
  s.last = reinterpret_cast<int32_t*>(b + l.off_last);
  s.run_ctr = reinterpret_cast<int64_t*>(b + l.run_ctr);
  s.run_off = reinterpret_cast<int64_t*>(b + l.run_off);
  s.run_child = reinterpret_cast<int32_t*>(b + l.run_child);
  s.run_page = reinterpret_cast<int32_t*>(b + l.run_page);
  s.run_bits = reinterpret_cast<uint32_t*>(b + l.run_bits);
  s.run_wpre = reinterpret_cast<uint32_t*>(b + l.run_wpre);
  s.run_ccnt = reinterpret_cast<uint32_t*>(b + l.run_ccnt);
  s.cmp_ring = reinterpret_cast<uint64_t*>(b + l.cmp_ring);
  s.cmp_bits = reinterpret_cast<uint32_t*>(b + l.cmp_bits);
  s.cmp_pre = reinterpret_cast<uint32_t*>(b + l.cmp_pre);
  s.cmp_ccnt = reinterpret_cast<uint32_t*>(b + l.cmp_ccnt);
  s.sp_ctr = reinterpret_cast<int64_t*>(b + l.sp_ctr);
  s.sp_req = reinterpret_cast<int32_t*>(b + l.sp_req);
  s.sp_ntok = reinterpret_cast<int32_t*>(b + l.sp_ntok);
  s.sp_m = reinterpret_cast<int32_t*>(b + l.sp_m);
  s.sp_h0 = reinterpret_cast<int64_t*>(b + l.sp_h0);
  s.sp_k = reinterpret_cast<int32_t*>(b + l.sp_k);
  s.sp_take = reinterpret_cast<int32_t*>(b + l.sp_take);
  s.sp_pinned = reinterpret_cast<int32_t*>(b + l.sp_pinned);
  s.sp_T = reinterpret_cast<int64_t*>(b + l.sp_T);
  s.sp_p0 = reinterpret_cast<int2*>(b + l.sp_p0);
  s.sp_fo = b + l.sp_fo;
  s.sp_first = reinterpret_cast<int32_t*>(b + l.sp_first);
  s.sp_late = reinterpret_cast<int32_t*>(b + l.sp_late);
  s.sp_wpg = reinterpret_cast<int32_t*>(b + l.sp_wpg);
  s.sp_wslot = reinterpret_cast<int32_t*>(b + l.sp_wslot);
  s.sp_wflag = b + l.sp_wflag;
  s.sp_victim = reinterpret_cast<int32_t*>(b + l.sp_victim);
  s.sp_vpos = reinterpret_cast<int32_t*>(b + l.sp_vpos);
  s.sp_wcnt = reinterpret_cast<int32_t*>(b + l.sp_wcnt);
  s.C = l.C;
  s.Q = l.Q;
  s.P = P;
  return s;
}

// --- field access ---------------------------------------------------------
__device__ __forceinline__ int32_t* ent_page(const BmState& s, int64_t i) {
  return reinterpret_cast<int32_t*>(s.ent + i * kEntBytes + 8);
}
__device__ __forceinline__ uint64_t* ent_key(const BmState& s, int64_t i) {
  return reinterpret_cast<uint64_t*>(s.ent + i * kEntBytes);
}
// a cached page's refcount, mirrored in its table entry so that a probe
// learns "found, and evictable?" from one load
__device__ __forceinline__ int32_t* ent_ref(const BmState& s, int64_t i) {
  return reinterpret_cast<int32_t*>(s.ent + i * kEntBytes + 12);
}
struct RecHead {
  int32_t ref, flag;
  uint32_t stamp;
  int32_t slot;
};
__device__ __forceinline__ RecHead rec_head(const BmState& s, int32_t p) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(s.rec + (int64_t)p * kRecBytes);
  return RecHead{(int32_t)v.x, (int32_t)v.y, v.z, (int32_t)v.w};
}
__device__ __forceinline__ int32_t* rec_ref(const BmState& s, int32_t p) {
  return reinterpret_cast<int32_t*>(s.rec + (int64_t)p * kRecBytes);
}
__device__ __forceinline__ int32_t* rec_flag(const BmState& s, int32_t p) {
  return reinterpret_cast<int32_t*>(s.rec + (int64_t)p * kRecBytes + 4);
}
__device__ __forceinline__ uint32_t* rec_stamp(const BmState& s, int32_t p) {
  return reinterpret_cast<uint32_t*>(s.rec + (int64_t)p * kRecBytes + 8);
}
__device__ __forceinline__ int32_t* rec_slot(const BmState& s, int32_t p) {
  return reinterpret_cast<int32_t*>(s.rec + (int64_t)p * kRecBytes + 12);
}
__device__ __forceinline__ uint64_t* rec_hash(const BmState& s, int32_t p) {
  return reinterpret_cast<uint64_t*>(s.rec + (int64_t)p * kRecBytes + 16);
}
__device__ __forceinline__ bool live(const RecHead& h, uint32_t stamp) {
  return (h.flag & 1) && h.ref == 0 && h.stamp == stamp;
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
  int32_t from_start;  // the tail kernel runs every op (a short step: no run, no speculation)
};

// Request metadata of a chunk of ops, staged in LDS.
struct OpMeta {
  int32_t op[kOpChunk];
  int32_t ntok[kOpChunk];
  int32_t nhash[kOpChunk];  // admits: page-hash count, -1 if it disagrees with ntok
  int64_t h0[kOpChunk];     // admits: index of the first page hash
};

// LDS of the step pass's admits: the pages taken for table positions below
// kBmThreads, and the table slots claimed by the current admit's inserts (a
// set, open addressing, -1 empty; cleared when each op ends).
struct AdmitLds {
  int32_t new_pg[kHeld * kBmThreads];
  int32_t claims[kSetSize];
};

// Per-workgroup scratch.
struct Shared {
  int32_t wave_sum[2][2][kBmWaves];  // block_rank2: [buffer][flag][wave]
  uint64_t evmask[kHeld][kBmWaves];  // probe: which held hits are evictable now
  // Per-op accumulators, two sets used by alternate ops: thread 0 clears the
  // previous op's set while the current op runs, so no clear can race with
  // an update of the op that uses the set.
  int32_t first_miss[2];
  int32_t count[2];
  int32_t tomb_reused[2];
  int64_t new_head;
};

__device__ __forceinline__ uint32_t slot_of(uint64_t h) { return (uint32_t)(h ^ (h >> 29)); }

// Values every lane holds alike but that come from LDS or a reduction: kept
// in scalar registers (VGPRs are the tail kernel's scarce resource).
__device__ __forceinline__ int32_t uni(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)((uint64_t)hi << 32 | lo);
}

// Adds x >= 0 to an LDS set of 2^kBits slots; false if it was already there
// (or the set is full: callers add at most half as many values as slots).
template <int kBits = 11>
__device__ __forceinline__ bool set_add(int32_t* set, int32_t x) {
  constexpr int kSize = 1 << kBits;
  uint32_t i = ((uint32_t)x * 2654435761u) >> (32 - kBits);
  for (int n = 0; n < kSize; ++n, i = (i + 1) & (kSize - 1)) {
    const int32_t prev = atomicCAS(&set[i], -1, x);
    if (prev == -1) return true;
    if (prev == x) return false;
  }
  return false;
}

__device__ __forceinline__ int32_t wave_min(int32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int32_t o = __shfl_xor(v, off);
    v = o < v ? o : v;
  }
  return v;
}
__device__ __forceinline__ int32_t wave_sum(int32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Block-wide exclusive ranks of two 0/1 flags (wavefront ballots + popcount,
// then the waves' totals through LDS); every thread gets both totals. One
// barrier per call: consecutive calls alternate between two LDS buffers
// (`buf` flips), and a buffer is rewritten only after the next call's barrier,
// which no thread passes before every thread has read it. Every thread must
// call it.
__device__ __forceinline__ void block_rank2(bool fa, bool fb, int32_t& ra, int32_t& rb,
                                            int32_t& ta, int32_t& tb, Shared& sh, int& buf) {
  const uint64_t ma = __ballot(fa), mb = __ballot(fb);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sh.wave_sum[buf][0][wave] = __popcll(ma);
    sh.wave_sum[buf][1][wave] = __popcll(mb);
  }
  __syncthreads();
  int32_t ba = 0, bb = 0, aa = 0, ab = 0;
#pragma unroll
  for (int w = 0; w < kBmWaves; ++w) {
    const int32_t ca = sh.wave_sum[buf][0][w], cb = sh.wave_sum[buf][1][w];
    ba += w < wave ? ca : 0;
    bb += w < wave ? cb : 0;
    aa += ca;
    ab += cb;
  }
  buf ^= 1;
  const uint64_t below = (1ull << lane) - 1ull;
  ra = ba + __popcll(ma & below);
  rb = bb + __popcll(mb & below);
  ta = uni(aa);
  tb = uni(ab);
}

// A lookup's result: the page under the key (or -1), the refcount mirrored in
// its entry, and the entry's slot — or, for a missing key, the first empty or
// tombstoned slot on its probe path, where it would be inserted.
struct Found {
  int32_t page, ref, slot;
  bool tomb;  // a miss's insertion slot is a tombstone
};

__device__ __forceinline__ int64_t tab_home(const BmState& s, uint64_t h) {
  return slot_of(h) & (s.C - 1);
}
__device__ __forceinline__ u32x4 tab_entry(const BmState& s, int64_t i) {
  return *reinterpret_cast<const u32x4*>(s.ent + i * kEntBytes);
}

// Looks up key h given the entry e at its home slot i (loaded by the caller, so
// that several lookups can have their first loads in flight together). Never
// runs concurrently with a writer of the table.
__device__ Found tab_find_at(const BmState& s, uint64_t h, int64_t i, u32x4 e) {
  const int64_t mask = s.C - 1;
  int64_t first_free = -1;
  for (int64_t n = 0; n < s.C; ++n) {
    if (n > 0) e = tab_entry(s, i);
    const int32_t v = (int32_t)e.z;
    if (v == kEmpty)
      return Found{-1, 0, (int32_t)(first_free >= 0 ? first_free : i), first_free >= 0};
    if (v >= 0 && ((uint64_t)e.y << 32 | e.x) == h) return Found{v, (int32_t)e.w, (int32_t)i, false};
    if (v == kTomb && first_free < 0) first_free = i;
    i = (i + 1) & mask;
  }
  return Found{-1, 0, (int32_t)first_free, first_free >= 0};
}

__device__ __forceinline__ Found tab_find(const BmState& s, uint64_t h) {
  const int64_t i = tab_home(s, h);
  return tab_find_at(s, h, i, tab_entry(s, i));
}

// Claims slot i for (h, page, refcount ref) if it still holds `expect` (empty
// or tombstone).
__device__ __forceinline__ bool tab_claim(const BmState& s, int64_t i, int32_t expect, uint64_t h,
                                          int32_t page, int32_t ref) {
  if (atomicCAS(ent_page(s, i), expect, kBusy) != expect) return false;
  *ent_key(s, i) = h;
  *ent_ref(s, i) = ref;
  *rec_slot(s, page) = (int32_t)i;
  __threadfence_block();
  __hip_atomic_store(ent_page(s, i), page, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return true;
}

// Inserts h -> page (other lanes may insert other keys at the same time) and
// records the slot in the page's record. Returns 1 if it reused a tombstone,
// 0 if it took an empty slot, -1 if the table was full (cannot happen: the
// load stays below 1/2 because of the rebuild threshold). `hint` is a slot on
// h's probe path at or before which nothing is free (from tab_find), or -1.
__device__ int32_t tab_insert(const BmState& s, uint64_t h, int32_t page, int32_t ref,
                              int64_t hint = -1) {
  const int64_t mask = s.C - 1;
  if (hint >= 0) {  // usually still free: one compare-and-swap
    if (tab_claim(s, hint, kEmpty, h, page, ref)) return 0;
    if (tab_claim(s, hint, kTomb, h, page, ref)) return 1;
  }
  int64_t i = slot_of(h) & mask;
  for (int64_t n = 0; n < 2 * s.C; ++n) {
    const int32_t v =
        __hip_atomic_load(ent_page(s, i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if ((v == kEmpty || v == kTomb) && tab_claim(s, i, v, h, page, ref))
      return v == kTomb ? 1 : 0;
    if (v == kEmpty || v == kTomb) continue;  // lost the race for this slot: look again
    i = (i + 1) & mask;
  }
  return -1;
}

// Counters every thread keeps in registers (all threads compute them alike).
struct Ctrs {
  int64_t free_top, head, tail, next_stamp, evictable, tombs, log_len;
};

// Moves the live ring entries [head, tail) to the front, in order.
__device__ void ring_compact(const BmArgs& a, Ctrs& c, Shared& sh, int& buf) {
  const BmState& s = a.s;
  const int64_t qm = s.Q - 1;
  int64_t out = c.head;
  for (int64_t base = c.head; base < c.tail; base += kBmThreads) {
    const int64_t pos = base + threadIdx.x;
    bool keep = false;
    uint64_t e = 0;
    if (pos < c.tail) {
      e = s.ring[pos & qm];
      keep = live(rec_head(s, (int32_t)(uint32_t)e), (uint32_t)(e >> 32));
    }
    // Every read of this chunk precedes the ranks' barrier. Writes go below
    // base + kBmThreads, where the later chunks no longer read.
    int32_t rank, unused_r, total, unused_t;
    block_rank2(keep, false, rank, unused_r, total, unused_t, sh, buf);
    if (keep) s.ring[(out + rank) & qm] = e;
    out += total;
  }
  c.tail = out;
}

// Rebuilds the hash table from the cached pages (drops every tombstone).
__device__ void tab_rebuild(const BmArgs& a, Ctrs& c) {
  const BmState& s = a.s;
  for (int64_t i = threadIdx.x; i < s.C; i += kBmThreads) *ent_page(s, i) = kEmpty;
  __syncthreads();
  for (int32_t p = threadIdx.x; p < s.P; p += kBmThreads)
    if (*rec_flag(s, p) & 1) tab_insert(s, *rec_hash(s, p), p, *rec_ref(s, p));
  __syncthreads();
  c.tombs = 0;
}

// A page taken for request r (from the free stack or by eviction): table index
// i < n_pages gets refcount 2 (parent and child), except a partial last page
// (1: the child copies it); otherwise it is the child's copy (refcount 1).
// The taker of the table's last page or of the copy reports it. Table pages
// below kBmThreads are also recorded in new_pg (LDS).
__device__ __forceinline__ void take_page(const BmArgs& a, int32_t r, int32_t p, int64_t i,
                                          int64_t n_pages, bool in_table, bool cow, int32_t* row,
                                          int32_t* new_pg) {
  if (in_table) {
    row[i] = p;
    if (i < kHeld * kBmThreads) new_pg[i] = p;
    const bool last = i == n_pages - 1;
    *rec_ref(a.s, p) = (cow && last) ? 1 : 2;
    if (last) {
      if (cow)
        a.cow_src[r] = p;
      else
        a.child_last[r] = p;
    }
  } else {
    *rec_ref(a.s, p) = 1;
    a.cow_dst[r] = p;
    a.child_last[r] = p;
  }
}

__device__ void admit(const BmArgs& a, int32_t r, int32_t n, int32_t nhash, int64_t h0,
                      const uint64_t (&hk)[kHeld], Ctrs& c, Shared& sh, AdmitLds& al, int& buf,
                      int par) {
  const BmState& s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m = nhash;
  const int64_t n_pages = (n + 15) / 16;
  const bool cow = (n & 15) != 0;
  int32_t* row = a.tables + (int64_t)r * a.tstride;
  if (nhash < 0 || n_pages > a.twidth) {
    if (tid == 0) {
      a.status[r] = kStBad;
      a.hits[r] = 0;
      a.child_last[r] = a.cow_src[r] = a.cow_dst[r] = -1;
      raise_err(a.err, MKV_DEVERR_BM);
    }
    return;
  }
  if (c.tombs > s.C / 4) tab_rebuild(a, c);

  // 1. probe every page hash (the first kHeld*kBmThreads from registers); a
  //    missing key remembers its insertion slot; evictable hits go into
  //    per-wave ballots. The free-stack entries this request may take are
  //    loaded meanwhile (one per thread).
  const int64_t may_take = n_pages + (cow ? 1 : 0);
  const int64_t pf_n = may_take < c.free_top ? may_take : c.free_top;
  const int32_t pf_page = tid < pf_n ? s.free_list[c.free_top - 1 - tid] : -1;
  // per held page: the probe's page (or -1), the mirrored refcount, and the
  // entry's slot (a hit) or the insertion slot (a miss)
  int32_t held_pg[kHeld], held_ref[kHeld], held_slot[kHeld];
  bool held_tomb[kHeld];
  int32_t miss = INT_MAX;
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int64_t i = tid + (int64_t)j * kBmThreads;
    held_pg[j] = -1;
    held_ref[j] = 1;
    held_slot[j] = -1;
    held_tomb[j] = false;
    if (i < m) {
      const Found f = tab_find(s, hk[j]);
      row[i] = f.page;
      held_pg[j] = f.page;
      held_ref[j] = f.page >= 0 ? f.ref : 1;
      held_slot[j] = f.slot;
      held_tomb[j] = f.tomb;
      if (f.page < 0 && (int32_t)i < miss) miss = (int32_t)i;
    }
  }
  for (int64_t i = tid + (int64_t)kHeld * kBmThreads; i < m; i += kBmThreads) {
    const int32_t p = tab_find(s, a.hashes[h0 + i]).page;
    row[i] = p;
    if (p < 0 && (int32_t)i < miss) miss = (int32_t)i;
  }
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const uint64_t em = __ballot(held_pg[j] >= 0 && held_ref[j] == 0);
    if (lane == 0) sh.evmask[j][wave] = em;
  }
  miss = wave_min(miss);
  if (lane == 0 && miss != INT_MAX) atomicMin(&sh.first_miss[par], miss);
  __syncthreads();
  const int64_t k = uni(sh.first_miss[par] < m ? sh.first_miss[par] : (int32_t)m);

  // 2. hits that are evictable now get pinned: count them for the OOM check
  //    (every thread adds up the ballots itself; hits past the held pages, if
  //    any, through one more reduction)
  //    (every lane reads all the wave ballots: LDS broadcasts)
  int32_t pinned_held = 0;
#pragma unroll
  for (int w = 0; w < kHeld * kBmWaves; ++w) {
    const int64_t first = (int64_t)(w / kBmWaves) * kBmThreads + (w % kBmWaves) * 64;
    if (first < k) {
      const uint64_t em = sh.evmask[w / kBmWaves][w % kBmWaves];
      pinned_held += __popcll(k - first >= 64 ? em : em & ((1ull << (k - first)) - 1ull));
    }
  }
  int64_t pinned = uni(pinned_held);
  if (k > (int64_t)kHeld * kBmThreads) {
    int32_t cnt = 0;
    for (int64_t i = tid + (int64_t)kHeld * kBmThreads; i < k; i += kBmThreads)
      cnt += *rec_ref(s, row[i]) == 0;
    cnt = wave_sum(cnt);
    if (lane == 0 && cnt) atomicAdd(&sh.count[par], cnt);
    __syncthreads();
    pinned += uni(sh.count[par]);
  }
  const int64_t take = n_pages - k + (cow ? 1 : 0);
  if (take > c.free_top + c.evictable - pinned) {
    if (tid == 0) {
      a.status[r] = kStOom;
      a.hits[r] = 0;
      a.child_last[r] = a.cow_src[r] = a.cow_dst[r] = -1;
    }
    return;
  }

  // 3. pin the hits, for the parent and the forked child at once (+2)
  //    (the owner of the table's last page, when it is a hit, also reports it
  //    as the child's last page: with a partial last page it is never a hit)
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int64_t i = tid + (int64_t)j * kBmThreads;
    if (i < k) {
      *rec_ref(s, held_pg[j]) = held_ref[j] + 2;
      *ent_ref(s, held_slot[j]) = held_ref[j] + 2;
      if (i == n_pages - 1) a.child_last[r] = held_pg[j];
    }
  }
  for (int64_t i = tid + (int64_t)kHeld * kBmThreads; i < k; i += kBmThreads) {
    const int32_t p = row[i];
    const RecHead h = rec_head(s, p);
    *rec_ref(s, p) = h.ref + 2;
    *ent_ref(s, h.slot) = h.ref + 2;
    if (i == n_pages - 1) a.child_last[r] = p;
  }
  c.evictable -= pinned;
  const int64_t from_free = take < c.free_top ? take : c.free_top;
  if (pinned > 0 && from_free < take) __syncthreads();  // pins land before liveness checks

  // 4. take pages: the free stack's top first, then LRU victims in order. The
  //    first n_pages-k go to the table (held by parent and child: refcount 2,
  //    except a partial last page, which the child copies: 1), the last (if
  //    any) is the child's copy (refcount 1).
  const int64_t table_new = n_pages - k;
  //    Whoever takes the table's last page or the child's copy reports it.
  for (int64_t j = tid; j < from_free; j += kBmThreads) {
    const int32_t p = j == tid ? pf_page : s.free_list[c.free_top - 1 - j];
    take_page(a, r, p, k + j, n_pages, table_new - j > 0, cow, row, al.new_pg);
  }
  c.free_top -= from_free;
  int64_t done = from_free;
  const int64_t qm = s.Q - 1;
  while (done < take) {
    if (c.head >= c.tail) {  // fewer live entries than counted: state is corrupt
      if (tid == 0) raise_err(a.err, MKV_DEVERR_BM);
      break;
    }
    // Nearly every entry at the LRU's old end is live, so a window of the
    // victims still wanted plus a little slack usually suffices: every entry
    // examined costs a scattered record load.
    const int64_t want = take - done;
    const int64_t fit = (want + 16 + 63) / 64 * 64;
    const int64_t win = fit < kBmThreads ? fit : kBmThreads;
    const int64_t pos = c.head + tid;
    bool ok = false;
    int32_t pg = 0;
    RecHead h{};
    if (tid < win && pos < c.tail) {
      const uint64_t e = s.ring[pos & qm];
      pg = (int32_t)(uint32_t)e;
      h = rec_head(s, pg);
      ok = live(h, (uint32_t)(e >> 32));
    }
    int32_t rank, unused_r, total, unused_t;
    block_rank2(ok, false, rank, unused_r, total, unused_t, sh, buf);
    if (ok && rank < want) {
      const int64_t j = done + rank;
      *ent_page(s, h.slot) = kTomb;  // the page's key leaves the table
      *rec_flag(s, pg) = h.flag & ~1;
      take_page(a, r, pg, k + j, n_pages, j < table_new, cow, row, al.new_pg);
      if (c.log_len + (j - from_free) < a.evict_cap)
        a.evict_log[c.log_len + (j - from_free)] = pg;
      if (rank == want - 1) sh.new_head = pos + 1;
    }
    __syncthreads();
    const int64_t got = total < want ? total : want;
    c.head = total >= want ? uni64(sh.new_head) : (c.head + win < c.tail ? c.head + win : c.tail);
    c.evictable -= got;
    c.tombs += got;
    done += got;
  }
  c.log_len += done - from_free;
  const bool evicted = done > from_free;

  // 5. register the new full pages' hashes unless already present. A key the
  //    probe did not find is still absent (only evictions ran since, and they
  //    only remove keys); a key it found is present unless its page was just
  //    evicted. All presence checks finish before any insert (barrier), so no
  //    check reads a page another lane is registering; the pages taken are
  //    read from LDS. A missing key goes to the insertion slot its probe found
  //    (still empty or a tombstone), claimed in LDS so that one lane writes it
  //    with plain stores; keys without a slot of their own are inserted after
  //    a barrier, by compare-and-swap.
  bool reg[kHeld];
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int64_t i = tid + (int64_t)j * kBmThreads;
    reg[j] = false;
    if (i < m && i >= k) {
      const int32_t seen = held_pg[j];
      reg[j] = seen < 0 ||
               (evicted && !((*rec_flag(s, seen) & 1) && *rec_hash(s, seen) == hk[j]));
    }
  }
  __syncthreads();
  int32_t reused = 0;
  bool later[kHeld];
  int32_t reg_pg[kHeld];
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    later[j] = false;
    reg_pg[j] = 0;
    if (!reg[j]) continue;
    const int32_t p = al.new_pg[tid + j * kBmThreads];  // j < kHeld: always in LDS
    reg_pg[j] = p;
    *rec_hash(s, p) = hk[j];
    *rec_flag(s, p) = 1;
    if (held_pg[j] < 0 && held_slot[j] >= 0 && set_add(al.claims, held_slot[j])) {
      *reinterpret_cast<u32x4*>(s.ent + (int64_t)held_slot[j] * kEntBytes) =
          u32x4{(uint32_t)hk[j], (uint32_t)(hk[j] >> 32), (uint32_t)p, 2u};
      *rec_slot(s, p) = held_slot[j];
      reused += held_tomb[j] ? 1 : 0;
    } else {
      later[j] = true;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kHeld; ++j)
    if (later[j]) reused += tab_insert(s, hk[j], reg_pg[j], 2) == 1;
  if (m > (int64_t)kHeld * kBmThreads) __syncthreads();  // the inserts above are complete
  // pages past the held ones (requests longer than kHeld*kBmThreads pages)
  for (int64_t base = (int64_t)kHeld * kBmThreads; base < m; base += kBmThreads) {
    const int64_t i = base + tid;
    bool rg = false;
    uint64_t h = 0;
    if (i < m && i >= k) {
      h = a.hashes[h0 + i];
      rg = tab_find(s, h).page < 0;
    }
    __syncthreads();
    if (rg) {
      const int32_t p = row[i];
      *rec_hash(s, p) = h;
      *rec_flag(s, p) = 1;
      reused += tab_insert(s, h, p, 2) == 1;
    }
    __syncthreads();
  }
  if (reused) atomicAdd(&sh.tomb_reused[par], reused);  // a few lanes: cheaper than a shuffle sum
  __syncthreads();
  c.tombs -= uni(sh.tomb_reused[par]);

  if (tid == 0) {  // the page-valued results were written by their owners
    a.hits[r] = (int32_t)k;
    a.status[r] = kStOk;
    if (!cow) {
      a.cow_src[r] = a.cow_dst[r] = -1;
      if (n_pages == 0) a.child_last[r] = -1;
    }
  }
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
__device__ void release(const BmArgs& a, int32_t r, int32_t n, Ctrs& c, Shared& sh, int& buf) {
  const BmState& s = a.s;
  const int64_t n_pages = n < 0 ? 0 : (n + 15) / 16;
  const bool cow = (n & 15) != 0;
  const int32_t* row = a.tables + (int64_t)r * a.tstride;
  // the first chunk's pages are loaded with the status, before it is known
  const int64_t j0 = threadIdx.x;
  const int32_t page0 = j0 < n_pages && n_pages <= a.twidth ? row[n_pages - 1 - j0] : 0;
  const int32_t st = a.status[r];
  const int32_t child = a.child_last[r];
  if (st != kStOk) {  // an OOM request holds nothing; anything else is a caller error
    if (st != kStOom && threadIdx.x == 0) raise_err(a.err, MKV_DEVERR_BM);
    return;
  }
  const int64_t qm = s.Q - 1;
  if (cow) {  // the child's private copy: uncached, refcount 1 -> free stack
    if (threadIdx.x == 0) {
      *rec_ref(s, child) = 0;
      s.free_list[c.free_top] = child;
    }
    c.free_top += 1;
  }
  if (c.tail - c.head + n_pages > s.Q) ring_compact(a, c, sh, buf);
  for (int64_t base = 0; base < n_pages; base += kBmThreads) {
    const int64_t j = base + threadIdx.x;  // j-th page from the tail
    bool to_lru = false, to_free = false;
    int32_t page = 0;
    if (j < n_pages) {
      const int64_t i = n_pages - 1 - j;
      page = base == 0 ? page0 : row[i];
      const RecHead h = rec_head(s, page);
      const int32_t left = h.ref - ((cow && i == n_pages - 1) ? 1 : 2);
      *rec_ref(s, page) = left;
      if (h.flag & 1) *ent_ref(s, h.slot) = left;
      if (left == 0) {
        to_lru = (h.flag & 1) != 0;
        to_free = !to_lru;
      }
    }
    int32_t rl, rf, n_lru, n_free;
    block_rank2(to_lru, to_free, rl, rf, n_lru, n_free, sh, buf);
    if (to_lru) {
      const uint32_t stamp = (uint32_t)(c.next_stamp + rl);
      s.ring[(c.tail + rl) & qm] = (uint32_t)page | (uint64_t)stamp << 32;
      *rec_stamp(s, page) = stamp;
    }
    if (to_free) s.free_list[c.free_top + rf] = page;
    c.tail += n_lru;
    c.next_stamp += n_lru;
    c.evictable += n_lru;
    c.free_top += n_free;
  }
  if (threadIdx.x == 0) a.status[r] = kStReleased;
}

// Loads the page hashes this thread holds for op t of the staged chunk.
__device__ __forceinline__ void fetch_hashes(const BmArgs& a, const OpMeta& om, int t,
                                             uint64_t (&h)[kHeld]) {
  const bool adm = om.op[t] >= 0;
  const int64_t nh = om.nhash[t], h0 = om.h0[t];
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int64_t i = threadIdx.x + (int64_t)j * kBmThreads;
    h[j] = adm && i < nh ? a.hashes[h0 + i] : 0;
  }
}

// ---------------------------------------------------------------------------
// Group admits: up to kGroup consecutive admits resolved from one round of
// loads.
//
// A single admit waits for several dependent memory round trips (its probe,
// the LRU window's ring entries and then their records, the liveness of the
// keys it registers), separated by barriers. A group issues those loads once
// for all its members, against the state S0 at the group's start, resolves
// the members in op order from registers and LDS, and writes the state once
// at the end. While a group resolves, global memory holds S0, except for
// evictions found past the preloaded LRU window, which are written at once:
// an evicted page has no other live ring entry, so no later read of the ring
// sees a difference.
//
// Thread i owns table position i of every member (members have at most
// kBmThreads pages). A page key hashes a request's whole prefix up to the end
// of that page, so a key occurs at one position only: which members share a
// key at position i (a class), and which of them hit it from the probe or
// registered it, is in thread i's own registers as 8-bit masks. What other
// threads need is in LDS: bitmaps over the pages evicted and pinned
// (refcount 0 in S0, then hit) in the group, the preloaded LRU window and
// free-stack top, the evicted pages handed to the positions that take them,
// and per member and position the probe result and the page it gets.
//
// Member u at position i, from S0's probe result p0 (page or -1):
//   present  = p0 >= 0 and not evicted in the group, or an earlier member of
//              its class registered the key (then that member's page);
//   k        = the first position not present;
//   pinned   = hits (< k) from the probe with refcount 0 in S0 that no earlier
//              member of the class hit (those are held already);
//   OOM      = take > free + evictable - pinned (then nothing changes);
//   takes    = the free stack's top, then the LRU window's oldest entries that
//              are live in S0 and not pinned in the group;
//   register = positions k..m-1 whose key is not present after the takes.
// Refcounts written at the end: a page hit from the probe gets its S0 count +
// 2 per member hitting it (written by the last of them); a taken page 2 (1
// for a partial last page, which the child copies) + 2 per later member
// hitting its registration; a copy-on-write page 1.
//
// The member loop is rolled (its code once, for the instruction cache) and
// reaches per-member data only through LDS and mask shifts; the set-up and
// write-back loops over members are unrolled and keep the keys, probe pages,
// slots and refcounts in registers.
// ---------------------------------------------------------------------------
constexpr int kGroup = 8;
constexpr int32_t kGroupMaxPages = 1 << 17;  // two page bitmaps in LDS, 16 KiB each
constexpr int kWin = 2 * kBmThreads;         // preloaded LRU window entries
constexpr int kFreePre = 2 * kBmThreads;     // preloaded free-stack entries
constexpr int kClaimBits = 12;               // LDS set of claimed table slots
constexpr int kGroupRegCap = (1 << kClaimBits) / 2;  // registrations per group, at most
constexpr int32_t kPinBit = 1 << 30;  // probe result: refcount 0 in S0 (pages < 2^28)
constexpr int32_t kTombBit = 1 << 30;  // a miss's insertion slot is a tombstone (slots < 2^30)
static_assert(kGroup <= 8, "a class mask is one byte per member");

struct GroupLds {
  uint32_t ev[kGroupMaxPages / 32];   // pages evicted in the group
  uint32_t pn[kGroupMaxPages / 32];   // pages pinned in the group
  int32_t probe[kGroup][kBmThreads];  // S0 probe: page | kPinBit, or -1
  int32_t page[kGroup][kBmThreads];   // the page a member's position gets
  int32_t win_pg[kWin];               // LRU window: the page if live in S0, else -1
  int32_t win_slot[kWin];             // the table slot of its key
  uint32_t win_ev[kWin / 32];         // window positions evicted
  int32_t fpre[kFreePre];             // free-stack entries from the top
  int32_t take_pg[kBmThreads + 2];    // one member's evicted pages, in take order
  int32_t claims[1 << kClaimBits];    // table slots claimed by registrations
  uint64_t pinmask[kGroup][kBmWaves];  // per member and wave: pinning hits
  int32_t wave_miss[kGroup][kBmWaves]; // per member and wave: the first miss
  int32_t hits[kGroup];  // per member: its hits, or -1 if it got OOM
  int32_t copy_pg[kGroup];
  int32_t reused;  // registrations that reused a tombstone
};

__device__ __forceinline__ bool bit_get(const uint32_t* b, int32_t p) {
  return (b[p >> 5] >> (p & 31)) & 1u;
}
__device__ __forceinline__ void bit_set(uint32_t* b, int32_t p) {
  atomicOr(&b[p >> 5], 1u << (p & 31));
}
// The members sharing member u's key at this position (its class, u excluded).
__device__ __forceinline__ uint32_t class_of(uint64_t cls, int u) {
  return (uint32_t)(cls >> (8 * u)) & 0xffu;
}

// The next kGroup ops' request metadata, staged in LDS by the group pass;
// a member is a valid admit of at most kBmThreads pages that fits its table.
struct GroupMeta {
  int32_t op[kGroup], ntok[kGroup], nhash[kGroup], ok[kGroup];
  int64_t h0[kGroup];
};

// Admits the g staged members (all eligible). Returns how many it processed: fewer when the registrations would outgrow the claim
// set, and the rest start the next group.
__device__ int group_admit(const BmArgs& a, const GroupMeta& om, int g, Ctrs& c, Shared& sh,
                           GroupLds& gl, int& buf) {
  static_assert(kWin == 2 * kBmThreads && kFreePre == 2 * kBmThreads, "two entries per thread");
  const BmState& s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i = tid;
  if (c.tombs > s.C / 4) tab_rebuild(a, c);
  // ring positions relative to head0 (a span is below Q < 2^31), free-stack
  // counts (below P) and registration counts fit 32 bits
  const int64_t head0 = c.head, log0 = c.log_len, qm = s.Q - 1;
  const int32_t span = (int32_t)(c.tail - head0), free0 = (int32_t)c.free_top;
  const int32_t wlen = span < kWin ? span : kWin;
  int32_t free_top = free0, evictable = (int32_t)c.evictable, pos = 0;
  int64_t log_len = log0, tombs = c.tombs;

  // 1. loads against S0: the members' page hashes, then their home entries;
  //    the LRU window's ring entries, then their records; the free stack's top
  int32_t mm[kGroup];
  uint64_t key[kGroup];
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    mm[u] = u < g ? uni(om.nhash[u]) : 0;
    key[u] = i < mm[u] ? a.hashes[om.h0[u] + i] : 0;
  }
  uint64_t went[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int32_t w = tid + j * kBmThreads;
    went[j] = w < wlen ? s.ring[(head0 + w) & qm] : 0;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int32_t t = tid + j * kBmThreads;
    if (t < free0) gl.fpre[t] = s.free_list[free0 - 1 - t];
  }
  u32x4 e0[kGroup];
#pragma unroll
  for (int u = 0; u < kGroup; ++u)
    e0[u] = i < mm[u] ? tab_entry(s, tab_home(s, key[u])) : u32x4{0u, 0u, 0u, 0u};
  RecHead wh[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int32_t w = tid + j * kBmThreads;
    wh[j] = w < wlen ? rec_head(s, (int32_t)(uint32_t)went[j]) : RecHead{0, 0, 0u, 0};
  }
  const int32_t nw = (s.P + 31) >> 5;
  for (int32_t w = tid; w < nw; w += kBmThreads) {
    gl.ev[w] = 0;
    gl.pn[w] = 0;
  }
  for (int w = tid; w < (1 << kClaimBits); w += kBmThreads) gl.claims[w] = -1;
  if (tid < kWin / 32) gl.win_ev[tid] = 0;
  if (tid == 0) gl.reused = 0;
  int32_t p0[kGroup], slot0[kGroup], ref0[kGroup];
  uint32_t mtomb = 0;  // bit u: the insertion slot of member u's key is a tombstone
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    p0[u] = -1;
    ref0[u] = 0;
    slot0[u] = -1;
    if (i < mm[u]) {
      const Found f = tab_find_at(s, key[u], tab_home(s, key[u]), e0[u]);
      p0[u] = f.page;
      ref0[u] = f.ref;
      slot0[u] = f.slot;
      mtomb |= f.tomb ? 1u << u : 0u;
    }
    if (u < g) gl.probe[u][i] = p0[u] < 0 ? -1 : (p0[u] | (ref0[u] == 0 ? kPinBit : 0));
  }
  uint64_t cls = 0;  // byte u: the members with member u's key here
#pragma unroll
  for (int u = 0; u < kGroup; ++u)
#pragma unroll
    for (int v = u + 1; v < kGroup; ++v)
      if (i < mm[u] && i < mm[v] && key[u] == key[v])
        cls |= 1ull << (8 * u + v) | 1ull << (8 * v + u);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int32_t w = tid + j * kBmThreads;
    if (w < wlen) {
      const int32_t p = (int32_t)(uint32_t)went[j];
      gl.win_pg[w] = live(wh[j], (uint32_t)(went[j] >> 32)) ? p : -1;
      gl.win_slot[w] = wh[j].slot;
    }
  }
  __syncthreads();

  // 2. the members in op order
  // idx-th entry from the S0 top. The global read is volatile so that it stays
  // a load of its own: merged with the LDS read into one flat load, it would
  // wait for every outstanding memory operation.
  auto free_at = [&](int32_t idx) -> int32_t {
    if (idx < kFreePre) return gl.fpre[idx];
    return *static_cast<const volatile int32_t*>(s.free_list + (free0 - 1 - idx));
  };
  // bit u at this position: member u hit from the probe / hit a registration
  // of its class / registers its key
  uint32_t mprobe = 0, mgroup = 0, mreg = 0;
  int done = 0;
  int32_t regs = 0;  // registrations so far, bounded from above
#pragma unroll 1
  for (int u = 0; u < g; ++u) {
    const int32_t m = uni(om.nhash[u]), n = uni(om.ntok[u]), r = uni(om.op[u]);
    if (u > 0 && regs + m > kGroupRegCap) break;
    const int32_t np = (n + 15) / 16;
    const bool cow = (n & 15) != 0;
    done = u + 1;
    const uint32_t bit = 1u << u, below = bit - 1u;
    const uint32_t ecls = class_of(cls, u);
    // hits
    int32_t pw = -1, cur = -1;
    bool from_probe = false;
    if (i < m) {
      pw = gl.probe[u][i];
      const uint32_t regd = ecls & mreg & below;
      if (pw >= 0 && !bit_get(gl.ev, pw & ~kPinBit)) {
        cur = pw & ~kPinBit;
        from_probe = true;
      } else if (regd) {
        cur = gl.page[__builtin_ctz(regd)][i];
      }
    }
    const bool pinnable = from_probe && (pw & kPinBit) && !(ecls & mprobe & below);
    // per wave: the first miss and the pinnable hits, from ballots
    const uint64_t mb = __ballot(i < m && cur < 0);
    const uint64_t pmask = __ballot(pinnable);
    if (lane == 0) {
      gl.pinmask[u][wave] = pmask;
      gl.wave_miss[u][wave] = mb ? wave * 64 + (int32_t)__builtin_ctzll(mb) : INT_MAX;
    }
    __syncthreads();
    int32_t k = m;
#pragma unroll
    for (int w = kBmWaves - 1; w >= 0; --w) {
      const int32_t x = gl.wave_miss[u][w];
      k = x < k ? x : k;
    }
    k = uni(k);
    int32_t pinned = 0;
#pragma unroll
    for (int w = 0; w < kBmWaves; ++w) {
      const uint64_t em = gl.pinmask[u][w];
      const int32_t lim = k - w * 64;
      pinned += lim <= 0 ? 0 : __popcll(lim >= 64 ? em : em & ((1ull << lim) - 1ull));
    }
    pinned = uni(pinned);
    const int32_t take = np - k + (cow ? 1 : 0);
    if (take > free_top + evictable - pinned) {  // OOM: nothing changes
      if (tid == 0) {
        gl.hits[u] = -1;
        a.status[r] = kStOom;
        a.hits[r] = 0;
        a.child_last[r] = a.cow_src[r] = a.cow_dst[r] = -1;
      }
      continue;
    }
    if (tid == 0) gl.hits[u] = k;
    regs += m - k;
    if (i < k) {
      if (from_probe)
        mprobe |= bit;
      else
        mgroup |= bit;
      if (pinnable) bit_set(gl.pn, cur);
    }
    evictable -= pinned;
    // takes: the free stack's top first (positions read their own page)
    const int32_t from_free = take < free_top ? take : free_top;
    const int32_t fbase = free0 - free_top;
    int32_t pgu = i < k ? cur : -1;
    if (i >= k && i < np && i - k < from_free) pgu = free_at(fbase + i - k);
    if (tid == 0) gl.copy_pg[u] = cow && take - 1 < from_free ? free_at(fbase + take - 1) : -1;
    free_top -= from_free;
    //        then LRU victims in order, handed to their positions through LDS
    const int32_t want_all = take - from_free;
    if (want_all > 0) {
      if (pinned > 0) __syncthreads();  // the pins are visible to the scan
      int32_t got_all = 0;
      while (got_all < want_all) {
        if (pos >= span) {  // fewer live entries than counted: state is corrupt
          if (tid == 0) raise_err(a.err, MKV_DEVERR_BM);
          break;
        }
        const int32_t want = want_all - got_all;
        const int32_t w = pos + tid;
        bool ok = false;
        int32_t vp = 0, vslot = 0;
        if (w < wlen) {
          vp = gl.win_pg[w];
          vslot = gl.win_slot[w];
          ok = vp >= 0 && !bit_get(gl.pn, vp);
        } else if (w < span) {  // past the preloaded window: from memory (still S0)
          const uint64_t e = s.ring[(head0 + w) & qm];
          vp = (int32_t)(uint32_t)e;
          const RecHead h = rec_head(s, vp);
          vslot = h.slot;
          ok = live(h, (uint32_t)(e >> 32)) && !bit_get(gl.pn, vp);
        }
        int32_t rank, unused_r, total, unused_t;
        block_rank2(ok, false, rank, unused_r, total, unused_t, sh, buf);
        if (ok && rank < want) {
          bit_set(gl.ev, vp);
          gl.take_pg[got_all + rank] = vp;
          if (w < wlen) {
            bit_set(gl.win_ev, (int32_t)w);
          } else {
            *ent_page(s, vslot) = kTomb;
            *rec_flag(s, vp) = 0;
            const int64_t li = log_len + got_all + rank;
            if (li < a.evict_cap) a.evict_log[li] = vp;
          }
          if (rank == want - 1) sh.new_head = w + 1;
        }
        __syncthreads();
        const int32_t got = total < want ? total : want;
        pos = total >= want ? uni((int32_t)sh.new_head) : (pos + kBmThreads < span ? pos + kBmThreads : span);
        got_all += got;
      }
      evictable -= got_all;
      tombs += got_all;
      log_len += got_all;
      const int32_t ti = i - k - from_free;
      if (i >= k && i < np && ti >= 0) pgu = ti < got_all ? gl.take_pg[ti] : -1;
      if (tid == 0 && cow && take - 1 >= from_free)
        gl.copy_pg[u] = take - 1 - from_free < got_all ? gl.take_pg[take - 1 - from_free] : -1;
    }
    // registrations: positions k..m-1 whose key is absent after the takes
    // (this member's eviction bits are visible: its scan ended with a barrier)
    if (i >= k && i < m && pgu >= 0) {
      const bool present = (pw >= 0 && !bit_get(gl.ev, pw & ~kPinBit)) || (ecls & mreg & below);
      if (!present) mreg |= bit;
    }
    if (i < np) gl.page[u][i] = pgu;
  }
  __syncthreads();  // the members' pages and results are visible

  // 3. write the state: tables, refcounts, results
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    if (u >= done) break;
    const int32_t k = uni(gl.hits[u]);
    if (k < 0) continue;
    const int32_t r = uni(om.op[u]), n = uni(om.ntok[u]);
    const int32_t np = (n + 15) / 16;
    const bool cow = (n & 15) != 0;
    const uint32_t bit = 1u << u, below = bit - 1u, above = ~(bit | below);
    const uint32_t ecls = class_of(cls, u);
    if (i < np) {
      const int32_t pgu = gl.page[u][i];
      a.tables[(int64_t)r * a.tstride + i] = pgu;
      if (mprobe & bit) {  // the last member of the class holding it writes the count
        if (!(ecls & mprobe & above)) {
          const int32_t ref = ref0[u] + 2 * (1 + __popc(ecls & mprobe & below));
          *rec_ref(s, p0[u]) = ref;
          *ent_ref(s, slot0[u]) = ref;
        }
      } else if (i >= k && pgu >= 0) {
        int32_t ref = (cow && i == np - 1) ? 1 : 2;
        if (mreg & bit) ref += 2 * __popc(ecls & mgroup & above);
        *rec_ref(s, pgu) = ref;
      }
      if (i == np - 1) {
        if (cow)
          a.cow_src[r] = pgu;
        else
          a.child_last[r] = pgu;
      }
    }
    if (tid == 0) {
      a.hits[r] = k;
      a.status[r] = kStOk;
      if (cow) {
        const int32_t cp = gl.copy_pg[u];
        a.cow_dst[r] = a.child_last[r] = cp;
        if (cp >= 0) *rec_ref(s, cp) = 1;
      } else {
        a.cow_src[r] = a.cow_dst[r] = -1;
        if (np == 0) a.child_last[r] = -1;
      }
    }
  }
  //    evictions from the preloaded window: the key leaves the table; the log
  //    follows window order (every eviction past the window came later)
  {
    const bool ea = tid < wlen && bit_get(gl.win_ev, tid);
    const bool eb = tid + kBmThreads < wlen && bit_get(gl.win_ev, tid + kBmThreads);
    int32_t ra, rb, ta, tb;
    block_rank2(ea, eb, ra, rb, ta, tb, sh, buf);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (!(j == 0 ? ea : eb)) continue;
      const int w = tid + j * kBmThreads;
      const int32_t p = gl.win_pg[w];
      *ent_page(s, gl.win_slot[w]) = kTomb;
      *rec_flag(s, p) = 0;
      const int64_t li = log0 + (j == 0 ? ra : ta + rb);
      if (li < a.evict_cap) a.evict_log[li] = p;
    }
  }
  __syncthreads();  // tombstones and cleared flags land before registrations
  //    registrations: the probe's slot for the key (its insertion slot, or
  //    the slot of its evicted entry), claimed in LDS; the rest by CAS
  int32_t reused = 0;
  uint32_t later = 0;
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    const uint32_t bit = 1u << u;
    if (!(mreg & bit)) continue;
    const int32_t p = gl.page[u][i];
    const int32_t ref = 2 + 2 * __popc(class_of(cls, u) & mgroup & ~((bit << 1) - 1u));
    *rec_hash(s, p) = key[u];
    *rec_flag(s, p) = 1;
    if (slot0[u] >= 0 && set_add<kClaimBits>(gl.claims, slot0[u])) {
      *reinterpret_cast<u32x4*>(s.ent + (int64_t)slot0[u] * kEntBytes) =
          u32x4{(uint32_t)key[u], (uint32_t)(key[u] >> 32), (uint32_t)p, (uint32_t)ref};
      *rec_slot(s, p) = slot0[u];
      reused += (p0[u] >= 0 || (mtomb & bit)) ? 1 : 0;
    } else {
      later |= bit;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {  // the keys that lost their slot
    const uint32_t bit = 1u << u;
    if (!(later & bit)) continue;
    const int32_t ref = 2 + 2 * __popc(class_of(cls, u) & mgroup & ~((bit << 1) - 1u));
    reused += tab_insert(s, key[u], gl.page[u][i], ref) == 1;
  }
  if (reused) atomicAdd(&gl.reused, reused);
  __syncthreads();
  c.free_top = free_top;
  c.head = head0 + pos;
  c.evictable = evictable;
  c.log_len = log_len;
  c.tombs = tombs - uni(gl.reused);
  return done;
}

// ---------------------------------------------------------------------------
// Bulk release of the step's leading run of release ops, on many CUs.
//
// Sequentially, release j walks L_j = [its child's private copy (if any),
// then its table from the last page], dropping references; a page that
// reaches zero is pushed at that moment (LRU ring if cached, free stack
// otherwise). Concatenate the walks into one list L. During a run references
// only fall, so a page reaches zero exactly at its last occurrence in L, and
// only if the run drops all of its references. One workgroup walking L is
// bound by how many scattered cache lines one CU can touch, so the run is
// retired by four passes before the speculation and the tail kernel run the
// remaining ops:
//   setup (the step's one-workgroup setup kernel): the run (leading valid
//     releases, at most kRunMaxOps ops and kRunMaxElems references), each
//     op's status, child copy and reference count, their prefix sums, room on
//     the ring, the counters the run starts from;
//   drop (many): every element subtracts its references from its page's
//     refcount and records its position as the page's last occurrence;
//   mark (many): an element is a zero-crossing iff it is its page's last
//     occurrence and the refcount is now 0 (bit arrays: to the ring / to the
//     free stack); a cached page's final refcount is mirrored into its entry;
//     each chunk's counts (per array, and before each bit word);
//   push (many, sharing its launch with the speculation's probe): every
//     crossing written at its place in L order (its chunk's offset is the sum
//     of the counts of the chunks before it, which each workgroup adds up
//     itself); the last-occurrence slots reset to -1; the counters and the
//     requests' statuses.
// No kernel waits for another workgroup; the launches order the passes.
// ---------------------------------------------------------------------------
constexpr int kRunThreads = 256;
constexpr int kRunWaves = kRunThreads / 64;
constexpr int kDropGrid = 512;   // drop: a workgroup takes kDropUnroll x kRunThreads elements at a time
constexpr int kDropUnroll = 2;
constexpr int kDropChunk = kDropUnroll * kRunThreads;
constexpr int kPassGrid = 1024;  // mark and push: a workgroup takes a chunk at a time
constexpr int kChunkWords = kRunChunk / 32;
static_assert(kRunChunk == kRunThreads, "a chunk is one element per thread");
static_assert(2 * kChunkWords <= kRunThreads, "a thread per bit word of a chunk");

// The LRU ring is compacted (on many CUs, inside the run kernels) when more
// than an eighth of its span is dead entries, and when a run's pushes might
// not fit. Dead entries accumulate as admits pin cached pages, and a dense
// ring lets an admit find its victims in one window. Live entries are
// exactly the evictable pages, and a run leaves them live. One thread of the
// setup kernel decides, on every path, and keeps the counters the push pass
// starts from (its workgroup 0 rewrites them while the others read).
constexpr int64_t kCompactMinDead = 1024;
// c: the counters at the step's start (as the setup kernel loaded them)
__device__ void run_counters(const BmState& s, const Ctrs& c, int64_t run_refs) {
  const int64_t span = c.tail - c.head, dead = span - c.evictable;
  const int64_t pushes = run_refs < s.P ? run_refs : s.P;  // at most one per page
  const bool pays = dead > kCompactMinDead && dead * 8 > span;
  s.run_ctr[kRunCompact] = pays || span + pushes > s.Q;
  s.run_ctr[kRunSpan] = span;
  s.run_ctr[kRunTail0] = c.tail;
  s.run_ctr[kRunStamp0] = c.next_stamp;
  s.run_ctr[kRunFree0] = c.free_top;
  s.run_ctr[kRunEvict0] = c.evictable;
}

__device__ __forceinline__ bool valid_release(const BmArgs& a, int32_t op) {
  return op < 0 && -(op + 1) < a.num_requests;
}

// LDS of the step's setup: the first kStageOps ops with their requests'
// metadata (the run's releases and the admits after them both lie there,
// loaded in one round); a set of request ids (open addressing) with each
// id's first op, for the run's releases and then for the admits; the run's
// element offsets.
constexpr int kStageOps = 2048;
static_assert(kStageOps >= 2 * kRunMaxOps, "the run and the admits after it");
struct SetupLds {
  int32_t op[kStageOps];
  int32_t ntok[kStageOps];    // the request's tokens (0 if the op names no request)
  int32_t status[kStageOps];  // releases: the request's status (kStBad if invalid)
  int32_t child[kStageOps];   // releases: the request's child_last
  int32_t m[kStageOps];       // admits: its page-hash count
  int64_t h0[kStageOps];      // admits: its first page hash
  uint32_t key[2 * kRunMaxOps], firsti[2 * kRunMaxOps];
  int64_t off[kRunMaxOps + 1];
  int64_t wave_tot[kBmWaves];
  int32_t cut;
};

// Stages ops [0, min(num_ops, kStageOps)) and their requests' metadata (every
// load depends only on its op) and loads the counters, all in one round.
__device__ void setup_stage(const BmArgs& a, SetupLds& sl, Ctrs& c) {
  constexpr int kPer = kStageOps / kBmThreads;
  const int nst = a.num_ops < kStageOps ? a.num_ops : kStageOps;
  c.free_top = a.s.ctr[kFreeTop];
  c.head = a.s.ctr[kHead];
  c.tail = a.s.ctr[kTail];
  c.next_stamp = a.s.ctr[kNextStamp];
  c.evictable = a.s.ctr[kEvictable];
  c.tombs = a.s.ctr[kTombs];
  c.log_len = 0;  // unused here
  int32_t op[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int j = threadIdx.x + u * kBmThreads;
    op[u] = j < nst ? a.ops[j] : 0;
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int j = threadIdx.x + u * kBmThreads;
    if (j >= nst) continue;
    const int32_t o = op[u], r = o >= 0 ? o : -(o + 1);
    const bool ok = r < a.num_requests;
    int32_t nt = 0, st = kStBad, ch = -1, m = 0;
    int64_t h0 = 0;
    if (ok) {
      nt = a.ntok[r];
      if (o < 0) {
        st = a.status[r];
        ch = a.child_last[r];
      } else {
        h0 = a.hash_off[r];
        m = (int32_t)(a.hash_off[r + 1] - h0);
      }
    }
    sl.op[j] = o;
    sl.ntok[j] = nt;
    sl.status[j] = st;
    sl.child[j] = ch;
    sl.m[j] = m;
    sl.h0[j] = h0;
  }
  __syncthreads();
}

// The run's part of the setup. Returns its op count (0: no run), alike in
// every thread.
__device__ int32_t run_setup(const BmArgs& a, const Ctrs& c0, SetupLds& sl) {
  constexpr int kOpt = kRunMaxOps / kBmThreads;  // consecutive ops per thread
  static_assert(kOpt * kBmThreads == kRunMaxOps, "ops split evenly over the threads");
  const BmState& s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int limit = a.num_ops < kRunMaxOps ? a.num_ops : kRunMaxOps;
  if (tid == 0) sl.cut = limit;
  for (int i = tid; i < 2 * kRunMaxOps; i += kBmThreads) {
    sl.key[i] = 0xffffffffu;
    sl.firsti[i] = 0xffffffffu;
  }
  __syncthreads();
  int32_t r[kOpt], st[kOpt], nt[kOpt], ch[kOpt];
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    const int32_t op = j < limit ? sl.op[j] : 0;
    r[u] = -(op + 1);
    st[u] = kStBad;
    nt[u] = 0;
    ch[u] = -1;
    if (j < limit) {
      // the run also ends at an admitted request whose token count no longer
      // fits its table (a caller error the tail kernel handles as before)
      bool ok = valid_release(a, op);
      if (ok) {
        st[u] = sl.status[j];
        nt[u] = sl.ntok[j];
        ch[u] = sl.child[j];
        ok = st[u] != kStOk || (nt[u] >= 0 && (nt[u] + 15) / 16 <= a.twidth);
      }
      if (!ok) atomicMin(&sl.cut, j);
    }
  }
  __syncthreads();
  int n = sl.cut;
  if (n < kRunMinOps) {
    if (tid == 0) {
      s.run_ctr[kRunOps] = 0;
      run_counters(s, c0, 0);
    }
    return 0;
  }
  // a request released twice: the earliest op releases; sequentially a later
  // one finds it released (a caller error) unless it got OOM (silent)
  uint32_t slot[kOpt];
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    slot[u] = 0;
    if (j < n) {
      uint32_t q = ((uint32_t)r[u] * 2654435761u) & (2 * kRunMaxOps - 1);
      for (;;) {  // at most n of 2 kRunMaxOps slots are taken
        const uint32_t prev = atomicCAS(&sl.key[q], 0xffffffffu, (uint32_t)r[u]);
        if (prev == 0xffffffffu || prev == (uint32_t)r[u]) break;
        q = (q + 1) & (2 * kRunMaxOps - 1);
      }
      atomicMin(&sl.firsti[q], (uint32_t)j);
      slot[u] = q;
    }
  }
  __syncthreads();
  int64_t cnt[kOpt], mine = 0;
  int32_t child[kOpt];
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    cnt[u] = 0;
    child[u] = -2;
    if (j < n) {
      if (sl.firsti[slot[u]] == (uint32_t)j && st[u] == kStOk) {
        const bool cow = (nt[u] & 15) != 0;
        child[u] = cow ? ch[u] : -1;
        cnt[u] = (nt[u] + 15) / 16 + (cow ? 1 : 0);
      } else if (st[u] != kStOom) {
        raise_err(a.err, MKV_DEVERR_BM);
      }
    }
    mine += cnt[u];
  }
  // exclusive prefix sum of the counts (thread totals, then within a thread)
  int64_t incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) sl.wave_tot[wave] = incl;
  __syncthreads();
  int64_t before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kBmWaves; ++w) {
    before += w < wave ? sl.wave_tot[w] : 0;
    total += sl.wave_tot[w];
  }
  int64_t at = before + incl - mine;
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    if (j < n) sl.off[j] = at;
    at += cnt[u];
  }
  if (tid == 0) sl.off[n] = total;
  __syncthreads();
  if (total > kRunMaxElems) {  // the longest prefix of ops that fits
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (sl.off[mid] <= kRunMaxElems) lo = mid; else hi = mid - 1;
    }
    n = lo;  // ops after it are the tail kernel's (it repeats any error bit)
  }
  if (n < kRunMinOps) {
    if (tid == 0) {
      s.run_ctr[kRunOps] = 0;
      run_counters(s, c0, 0);
    }
    return 0;
  }
  for (int j = tid; j <= n; j += kBmThreads) s.run_off[j] = sl.off[j];
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    if (j < n) s.run_child[j] = child[u];
  }
  if (tid == 0) {
    s.run_ctr[kRunOps] = n;
    s.run_ctr[kRunTotal] = sl.off[n];
    run_counters(s, c0, sl.off[n]);
  }
  return n;
}

// The run's per-op tables, staged in a pass workgroup's LDS.
struct RunOps {
  int64_t off[kRunMaxOps + 1];
  int32_t child[kRunMaxOps];
  int32_t req[kRunMaxOps];
  int32_t np[kRunMaxOps];
};

__device__ __forceinline__ void run_stage(const BmArgs& a, int n, RunOps& ro) {
  for (int j = threadIdx.x; j <= n; j += kRunThreads) ro.off[j] = a.s.run_off[j];
  for (int j = threadIdx.x; j < n; j += kRunThreads) {
    ro.child[j] = a.s.run_child[j];
    const int32_t r = -(a.ops[j] + 1);
    ro.req[j] = r;
    ro.np[j] = (a.ntok[r] + 15) / 16;
  }
  __syncthreads();
}

// Element e of the run: its page and the references it drops. Its op is the
// last one starting at or before e (ops without elements share offsets).
__device__ __forceinline__ void run_elem(const BmArgs& a, const RunOps& ro, int n, int64_t e,
                                         int32_t& page, int32_t& drop) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ro.off[mid] <= e) lo = mid; else hi = mid - 1;
  }
  const int j = lo;
  const int32_t child = ro.child[j];
  const int64_t np = ro.np[j];
  const int64_t idx = e - ro.off[j] - (child >= 0 ? 1 : 0);
  const int64_t i = idx < 0 ? 0 : np - 1 - idx;  // the child's element loads a valid entry
  const int32_t tp = a.tables[(int64_t)ro.req[j] * a.tstride + i];
  page = idx < 0 ? child : tp;
  drop = idx < 0 ? 1 : ((child >= 0 && i == np - 1) ? 1 : 2);
}

__global__ __launch_bounds__(kRunThreads) void run_drop_kernel(BmArgs a) {
  __shared__ RunOps ro;
  const BmState& s = a.s;
  const int n = (int)s.run_ctr[kRunOps];
  const int64_t total = s.run_ctr[kRunTotal];
  if (n < kRunMinOps || (int64_t)blockIdx.x * kDropChunk >= total) return;
  run_stage(a, n, ro);
  for (int64_t c0 = (int64_t)blockIdx.x * kDropChunk; c0 < total;
       c0 += (int64_t)gridDim.x * kDropChunk) {
    int32_t pg[kDropUnroll], dr[kDropUnroll];
#pragma unroll
    for (int u = 0; u < kDropUnroll; ++u) {
      const int64_t e = c0 + u * kRunThreads + threadIdx.x;
      run_elem(a, ro, n, e < total ? e : total - 1, pg[u], dr[u]);
    }
#pragma unroll
    for (int u = 0; u < kDropUnroll; ++u) {
      const int64_t e = c0 + u * kRunThreads + threadIdx.x;
      if (e < total) {
        s.run_page[e] = pg[u];
        __hip_atomic_fetch_add(rec_ref(s, pg[u]), -dr[u], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_max(&s.last[pg[u]], (int32_t)e, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// A chunk's per-word set bits (wc[k][w], filled by the waves' lane 0) become
// each word's count before it within the chunk (pre[k]) and the chunk's
// total (ccnt[k]), for NB arrays; barriers before and after.
template <int NB>
__device__ __forceinline__ void chunk_counts(uint32_t (&wc)[2][kChunkWords], int64_t c,
                                             uint32_t* const (&pre)[NB],
                                             uint32_t* const (&ccnt)[NB]) {
  __syncthreads();
  if (threadIdx.x < NB * kChunkWords) {
    const int k = threadIdx.x / kChunkWords, w = threadIdx.x % kChunkWords;
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int v = 0; v < kChunkWords; ++v) {
      const uint32_t x = wc[k][v];
      before += v < w ? x : 0;
      all += x;
    }
    pre[k][c * kChunkWords + w] = before;
    if (w == 0) ccnt[k][c] = all;
  }
  __syncthreads();  // wc is rewritten by the next chunk
}

__global__ __launch_bounds__(kRunThreads) void run_mark_kernel(BmArgs a) {
  __shared__ uint32_t wc[2][kChunkWords];
  const BmState& s = a.s;
  const int n = (int)s.run_ctr[kRunOps];
  const int64_t total = n < kRunMinOps ? 0 : s.run_ctr[kRunTotal];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  {
    uint32_t* const pre[2] = {s.run_wpre, s.run_wpre + kRunMaxWords};
    uint32_t* const ccnt[2] = {s.run_ccnt, s.run_ccnt + kRunMaxChunks};
    for (int64_t c = blockIdx.x; c * kRunChunk < total; c += gridDim.x) {
      const int64_t e = c * kRunChunk + threadIdx.x;  // a wave: 64 aligned elements
      const int32_t pg = s.run_page[e < total ? e : total - 1];
      const RecHead h = rec_head(s, pg);
      const bool is_last = e < total && s.last[pg] == (int32_t)e;
      const bool zero = is_last && h.ref == 0;
      const bool cached = (h.flag & 1) != 0;
      if (is_last && cached) *ent_ref(s, h.slot) = h.ref;
      const uint64_t ml = __ballot(is_last), mr = __ballot(zero && cached),
                     mf = __ballot(zero && !cached);
      if (lane == 0) {
        const int wi = wave * 2;  // the wave's first word in the chunk
        wc[0][wi] = __popc((uint32_t)mr);
        wc[0][wi + 1] = __popc((uint32_t)(mr >> 32));
        wc[1][wi] = __popc((uint32_t)mf);
        wc[1][wi + 1] = __popc((uint32_t)(mf >> 32));
        if (e < total) {
          const int64_t w = e >> 5;
          uint32_t* b = s.run_bits;
          b[w] = (uint32_t)mr;
          b[w + 1] = (uint32_t)(mr >> 32);
          b[kRunMaxWords + w] = (uint32_t)mf;
          b[kRunMaxWords + w + 1] = (uint32_t)(mf >> 32);
          b[2 * kRunMaxWords + w] = (uint32_t)ml;
          b[2 * kRunMaxWords + w + 1] = (uint32_t)(ml >> 32);
        }
      }
      chunk_counts<2>(wc, c, pre, ccnt);
    }
  }
  // Compaction: the ring span [head, tail) is copied out, with a bit per entry
  // that stays live (an entry of a page this run pushes again does not).
  if (s.run_ctr[kRunCompact] == 0) return;
  const int64_t head = s.ctr[kHead], span = s.run_ctr[kRunSpan], qm = s.Q - 1;
  uint32_t* const pre[1] = {s.cmp_pre};
  uint32_t* const ccnt[1] = {s.cmp_ccnt};
  for (int64_t c = blockIdx.x; c * kRunChunk < span; c += gridDim.x) {
    const int64_t i = c * kRunChunk + threadIdx.x;  // a wave: 64 aligned entries
    bool keep = false;
    if (i < span) {
      const uint64_t e = s.ring[(head + i) & qm];
      const int32_t pg = (int32_t)(uint32_t)e;
      s.cmp_ring[i] = e;
      keep = live(rec_head(s, pg), (uint32_t)(e >> 32)) && (n < kRunMinOps || s.last[pg] < 0);
    }
    const uint64_t m = __ballot(keep);
    if (lane == 0) {
      const int wi = wave * 2;
      wc[0][wi] = __popc((uint32_t)m);
      wc[0][wi + 1] = __popc((uint32_t)(m >> 32));
      if (i < span) {
        s.cmp_bits[i >> 5] = (uint32_t)m;
        s.cmp_bits[(i >> 5) + 1] = (uint32_t)(m >> 32);
      }
    }
    chunk_counts<1>(wc, c, pre, ccnt);
  }
}

// The sum of cnt[lo, hi) over the workgroup (every thread gets it), two
// arrays at once; red is LDS for the waves' partial sums.
__device__ __forceinline__ void range_sum2(const uint32_t* c0, const uint32_t* c1, int64_t lo,
                                           int64_t hi, int64_t (&red)[2][kRunWaves],
                                           int64_t& t0, int64_t& t1) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t v0 = 0, v1 = 0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kRunThreads) {
    v0 += c0[i];
    v1 += c1 ? c1[i] : 0;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    v0 += __shfl_xor(v0, off);
    v1 += __shfl_xor(v1, off);
  }
  if (lane == 0) {
    red[0][wave] = v0;
    red[1][wave] = v1;
  }
  __syncthreads();
  t0 = t1 = 0;
#pragma unroll
  for (int w = 0; w < kRunWaves; ++w) {
    t0 += red[0][w];
    t1 += red[1][w];
  }
  __syncthreads();  // red is rewritten by the next sum
}

__device__ void spec_probe(const BmArgs& a, int32_t wg, int32_t nwg);

// Workgroups [0, kPassGrid) push the run; the rest run the speculation's probe
// (it reads only the table, which the push does not touch, and the setup's
// admit list).
__global__ __launch_bounds__(kRunThreads) void run_push_kernel(BmArgs a) {
  __shared__ int64_t red[2][kRunWaves];
  if (blockIdx.x >= kPassGrid) {
    spec_probe(a, blockIdx.x - kPassGrid, gridDim.x - kPassGrid);
    return;
  }
  const BmState& s = a.s;
  const int n = (int)s.run_ctr[kRunOps];
  const int64_t total = n < kRunMinOps ? 0 : s.run_ctr[kRunTotal];
  const bool cmp = s.run_ctr[kRunCompact] != 0;
  const int64_t head = s.ctr[kHead], span = s.run_ctr[kRunSpan], qm = s.Q - 1;
  const int64_t nch = (total + kRunChunk - 1) / kRunChunk;
  const int64_t ncc = cmp ? (span + kRunChunk - 1) / kRunChunk : 0;
  const int64_t b = blockIdx.x;
  if (b != 0 && b >= nch && b >= ncc && b * kRunThreads >= n) return;
  for (int64_t j = b * kRunThreads + threadIdx.x; j < (n >= kRunMinOps ? n : 0);
       j += (int64_t)kPassGrid * kRunThreads)
    if (s.run_child[j] != -2) a.status[-(a.ops[j] + 1)] = kStReleased;
  int64_t t0, t1;
  // the kept entries, from the head in order
  int64_t n_kept = 0;
  if (cmp) {
    range_sum2(s.cmp_ccnt, nullptr, 0, ncc, red, n_kept, t1);
    int64_t before;
    range_sum2(s.cmp_ccnt, nullptr, 0, b < ncc ? b : ncc, red, before, t1);
    for (int64_t c = b; c < ncc; c += kPassGrid) {
      const int64_t i = c * kRunChunk + threadIdx.x;
      if (i < span) {
        const uint32_t bits = s.cmp_bits[i >> 5], bit = 1u << (i & 31);
        if (bits & bit)
          s.ring[(head + before + s.cmp_pre[i >> 5] + __popc(bits & (bit - 1u))) & qm] =
              s.cmp_ring[i];
      }
      const int64_t next = c + kPassGrid < ncc ? c + kPassGrid : ncc;
      range_sum2(s.cmp_ccnt, nullptr, c, next, red, t0, t1);
      before += t0;
    }
  }
  // pushes go after the kept entries (compacted from the head) or the tail
  const int64_t tail0 = cmp ? head + n_kept : s.run_ctr[kRunTail0];
  const int64_t stamp0 = s.run_ctr[kRunStamp0], free0 = s.run_ctr[kRunFree0];
  const uint32_t* bw = s.run_bits;
  const uint32_t *cl = s.run_ccnt, *cf = s.run_ccnt + kRunMaxChunks;
  int64_t bl, bf;
  range_sum2(cl, cf, 0, b < nch ? b : nch, red, bl, bf);
  for (int64_t c = b; c < nch; c += kPassGrid) {
    const int64_t e = c * kRunChunk + threadIdx.x;
    const int64_t w = e >> 5;
    const uint32_t bit = 1u << (e & 31), below = bit - 1u;
    const uint32_t br = e < total ? bw[w] : 0u, bfw = e < total ? bw[kRunMaxWords + w] : 0u,
                   bl_w = e < total ? bw[2 * kRunMaxWords + w] : 0u;
    if ((br | bfw | bl_w) & bit) {
      const int32_t pg = s.run_page[e];
      if (bl_w & bit) s.last[pg] = -1;
      if (br & bit) {
        const int64_t rank = bl + s.run_wpre[w] + __popc(br & below);
        const uint32_t stamp = (uint32_t)(stamp0 + rank);
        s.ring[(tail0 + rank) & qm] = (uint32_t)pg | (uint64_t)stamp << 32;
        *rec_stamp(s, pg) = stamp;
      }
      if (bfw & bit) {
        const int64_t rank = bf + s.run_wpre[kRunMaxWords + w] + __popc(bfw & below);
        s.free_list[free0 + rank] = pg;
      }
    }
    const int64_t next = c + kPassGrid < nch ? c + kPassGrid : nch;
    range_sum2(cl, cf, c, next, red, t0, t1);
    bl += t0;
    bf += t1;
  }
  if (b == 0) {  // the counters after the run, and the speculation's starting point
    int64_t n_lru, n_free;
    range_sum2(cl, cf, 0, nch, red, n_lru, n_free);
    if (threadIdx.x == 0) {
      const int64_t ev = s.run_ctr[kRunEvict0] + n_lru, fr = free0 + n_free;
      s.ctr[kTail] = tail0 + n_lru;
      s.ctr[kNextStamp] = stamp0 + n_lru;
      s.ctr[kEvictable] = ev;
      s.ctr[kFreeTop] = fr;
      s.sp_ctr[kSpF] = fr;
      s.sp_ctr[kSpLive] = ev;
      s.sp_ctr[kSpHead] = head;
    }
  }
}

// ---------------------------------------------------------------------------
// Speculative resolution of a step's admits, on many CUs.
//
// The admits after the release run (up to kSpecOps valid admits of at most
// kSpecPos pages, distinct requests) are resolved together against the state
// S at the step's start, modelling exactly what earlier admits of the step do
// to later ones in the common case:
//   - a key absent at S is a hit for every admit after the first one holding
//     it (that one registers it: its first occurrence);
//   - a page hit at refcount 0 is pinned by the first admit hitting it;
//   - takes come in op order: the free stack's top, then the LRU's oldest
//     entries that are live at S and pinned by no admit of the step.
// Each admit is then checked for what this does not model:
//   - an OOM (against running free / evictable counts);
//   - a hit on, or a key it would register again after, a page that an
//     earlier admit (or, past its hits, itself) evicts;
//   - an LRU entry pinned in the step that an earlier admit's takes reach
//     (sequentially it would be that admit's victim);
//   - a window or first-occurrence table too small.
// The admits before the first violation are exactly what the sequential order
// gives, and are committed on many CUs; the tail kernel takes the rest.
//
// Refcounts: a hit adds 2 (parent and child), a taken page its base (2, 1
// for a partial last page the child copies, 1 for a copy-on-write page), by
// atomic adds: every page it takes is at refcount 0 at S. A last pass copies
// the cached pages' counts into their table entries.
// ---------------------------------------------------------------------------
constexpr int kSpecThreads = 512;
constexpr int kSpecGrid = 1024;
constexpr int kPosPer = kSpecPos / kSpecThreads;  // positions per thread
static_assert(kPosPer * kSpecThreads == kSpecPos, "positions split evenly over the threads");

__device__ __forceinline__ uint64_t* fo_key(const BmState& s, int64_t i) {
  return reinterpret_cast<uint64_t*>(s.sp_fo + i * 16);
}
__device__ __forceinline__ int32_t* fo_first(const BmState& s, int64_t i) {
  return reinterpret_cast<int32_t*>(s.sp_fo + i * 16 + 8);
}
__device__ __forceinline__ int32_t* spec_bad(const BmState& s) {
  return reinterpret_cast<int32_t*>(s.sp_ctr + kSpBad);  // the value fits 32 bits
}

// Records key h (absent at S) as held at occurrence code = admit * kSpecPos +
// position; the table keeps the smallest code. False if h is 0 (the empty key)
// or its probe runs past kFoMaxProbe slots.
__device__ bool fo_insert(const BmState& s, uint64_t h, int32_t code) {
  if (h == 0) return false;
  int64_t i = slot_of(h) & (kFoCap - 1);
  for (int n = 0; n < kFoMaxProbe; ++n, i = (i + 1) & (kFoCap - 1)) {
    const unsigned long long prev = atomicCAS(reinterpret_cast<unsigned long long*>(fo_key(s, i)),
                                              0ull, (unsigned long long)h);
    if (prev == 0ull || prev == h) {
      atomicMin(fo_first(s, i), code);
      return true;
    }
  }
  return false;
}

// The first occurrence code of key h (INT_MAX if none), after every insert.
__device__ int32_t fo_find(const BmState& s, uint64_t h) {
  int64_t i = slot_of(h) & (kFoCap - 1);
  for (int n = 0; n < kFoMaxProbe; ++n, i = (i + 1) & (kFoCap - 1)) {
    const uint64_t k = *fo_key(s, i);
    if (k == h) return *fo_first(s, i);
    if (k == 0) return INT_MAX;
  }
  return INT_MAX;
}

// The t-th page the step's admits take, in op order (victims past the window
// cannot belong to a committed admit: the scan marks the first admit lacking
// one as a violation; the bound only keeps a broken state in range).
__device__ __forceinline__ int32_t spec_take_at(const BmState& s, int64_t t, int64_t F) {
  const int64_t v = t - F;
  return t < F ? s.free_list[F - 1 - t] : s.sp_victim[v < kSpecWin ? v : kSpecWin - 1];
}

// tab_insert for inserts from many workgroups at once (one kernel that does
// nothing else with the table): a slot is claimed by a device-scope
// compare-and-swap of its page field straight to the page, and the key and
// refcount follow with plain stores; nothing in the kernel reads a key, and
// the next kernel sees them all.
__device__ int32_t tab_insert_dev(const BmState& s, uint64_t h, int32_t page, int32_t ref,
                                  int64_t hint) {
  const int64_t mask = s.C - 1;
  auto claim = [&](int64_t i, int32_t expect) -> bool {
    if (atomicCAS(ent_page(s, i), expect, page) != expect) return false;
    *ent_key(s, i) = h;
    *ent_ref(s, i) = ref;
    *rec_slot(s, page) = (int32_t)i;
    return true;
  };
  if (hint >= 0) {
    if (claim(hint, kEmpty)) return 0;
    if (claim(hint, kTomb)) return 1;
  }
  int64_t i = slot_of(h) & mask;
  for (int64_t n = 0; n < 2 * s.C; ++n) {
    const int32_t v =
        __hip_atomic_load(ent_page(s, i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v == kEmpty || v == kTomb) {
      if (claim(i, v)) return v == kTomb ? 1 : 0;
      continue;  // claimed by another workgroup meanwhile: read the slot again
    }
    i = (i + 1) & mask;
  }
  return -1;
}

// The first-occurrence table and the per-page first pinner, evicting admit
// and late holder are all-empty between steps: cleared once at init and by
// the finish kernel of every step that used them, on many CUs.
__device__ __forceinline__ void spec_clear_scratch(const BmState& s, int64_t g, int64_t stride) {
  for (int64_t i = g; i < kFoCap; i += stride)
    *reinterpret_cast<u32x4*>(s.sp_fo + i * 16) = u32x4{0u, 0u, (uint32_t)INT_MAX, 0u};
  for (int64_t p = g; p < s.P; p += stride) {
    s.sp_first[p] = INT_MAX;
    s.sp_late[p] = INT_MAX;
  }
}

// 1. The admits to speculate: the leading valid admits after the release run
//    (at most kSpecOps, of at most kSpecPos pages), cut before a request that
//    repeats; their metadata. The counters they start from come from the
//    push pass, after the run.
__device__ void spec_setup(const BmArgs& a, int32_t start, SetupLds& sl) {
  constexpr int kOpt = kSpecOps / kSpecThreads;
  static_assert(kOpt * kSpecThreads == kSpecOps, "ops split evenly over the threads");
  static_assert(kSpecOps == kRunMaxOps && kSpecThreads == kBmThreads, "the run's set and threads");
  const BmState& s = a.s;
  const int tid = threadIdx.x;
  const int32_t left = a.num_ops - start;
  const int limit = left < kSpecOps ? left : kSpecOps;
  __syncthreads();  // the run's reads of the set are done
  if (tid == 0) sl.cut = limit;
  for (int i = tid; i < 2 * kSpecOps; i += kSpecThreads) {
    sl.key[i] = 0xffffffffu;
    sl.firsti[i] = 0xffffffffu;
  }
  __syncthreads();
  int32_t r[kOpt], n[kOpt], m[kOpt];
  int64_t h0[kOpt];
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    r[u] = -1;
    n[u] = m[u] = 0;
    h0[u] = 0;
    if (j >= limit) continue;
    const int32_t op = sl.op[start + j];  // start + j < kStageOps: start <= kRunMaxOps
    bool ok = op >= 0 && op < a.num_requests;
    if (ok) {
      r[u] = op;
      n[u] = sl.ntok[start + j];
      h0[u] = sl.h0[start + j];
      const int64_t mm = sl.m[start + j], np = ((int64_t)n[u] + 15) / 16;
      ok = n[u] >= 0 && mm == n[u] / 16 && np <= a.twidth && np <= kSpecPos;
      m[u] = (int32_t)mm;
    }
    if (!ok) atomicMin(&sl.cut, j);
  }
  __syncthreads();
  const int lim2 = sl.cut;
  // a request admitted twice: the speculation stops before the second
  uint32_t slot[kOpt];
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    slot[u] = 0;
    if (j >= lim2) continue;
    uint32_t q = ((uint32_t)r[u] * 2654435761u) & (2 * kSpecOps - 1);
    for (;;) {  // at most kSpecOps of 2 kSpecOps slots are taken
      const uint32_t prev = atomicCAS(&sl.key[q], 0xffffffffu, (uint32_t)r[u]);
      if (prev == 0xffffffffu || prev == (uint32_t)r[u]) break;
      q = (q + 1) & (2 * kSpecOps - 1);
    }
    atomicMin(&sl.firsti[q], (uint32_t)j);
    slot[u] = q;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    if (j < lim2 && sl.firsti[slot[u]] != (uint32_t)j) atomicMin(&sl.cut, j);
  }
  __syncthreads();
  const int nspec = sl.cut;
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    if (j >= nspec) continue;
    s.sp_req[j] = r[u];
    s.sp_ntok[j] = n[u];
    s.sp_m[j] = m[u];
    s.sp_h0[j] = h0[u];
  }
  if (tid == 0) {
    s.sp_ctr[kSpN] = nspec;
    s.sp_ctr[kSpBad] = nspec;
    s.sp_ctr[kSpWin] = 0;
    s.sp_ctr[kSpReused] = 0;
    s.run_ctr[kRunNext] = start;
  }
}

// The step's setup, one workgroup: the table rebuilt when tombstones pass a
// quarter of it (no pass of the step holds a slot across this launch), the
// release run's setup, then the admits after the run.
__global__ __launch_bounds__(kBmThreads) void step_setup_kernel(BmArgs a) {
  __shared__ SetupLds sl;
  Ctrs c;
  setup_stage(a, sl, c);  // ends with a barrier, after every thread read the counters
  if (c.tombs > a.s.C / 4) {
    tab_rebuild(a, c);  // ends with a barrier
    if (threadIdx.x == 0) a.s.ctr[kTombs] = 0;
  }
  const int32_t start = run_setup(a, c, sl);
  spec_setup(a, start, sl);
}

// 2. Every speculated admit's page hashes looked up at S (a workgroup per
//    admit, in the push pass's launch); keys absent at S enter the
//    first-occurrence table.
__device__ void spec_probe(const BmArgs& a, int32_t wg, int32_t nwg) {
  const BmState& s = a.s;
  const int32_t n = (int32_t)s.sp_ctr[kSpN];
  for (int32_t j = wg; j < n; j += nwg) {
    const int32_t m = s.sp_m[j];
    const int64_t h0 = s.sp_h0[j];
    int2* out = s.sp_p0 + (int64_t)j * kSpecPos;
    for (int32_t i = threadIdx.x; i < m; i += blockDim.x) {
      const uint64_t h = a.hashes[h0 + i];
      const Found f = tab_find(s, h);
      if (f.page >= 0) {
        out[i] = int2{f.page | (f.ref == 0 ? kPinBit : 0), f.slot};
      } else {
        out[i] = int2{-1, f.slot | (f.tomb ? kTombBit : 0)};
        if (!fo_insert(s, h, j * kSpecPos + i)) atomicMin(spec_bad(s), j);
      }
    }
  }
}

// 3. Per admit: its hits (a key absent at S is present if an earlier admit
//    holds it: the position records that occurrence), its takes, and the
//    first admit pinning each page it hits at refcount 0. An admit holding a
//    key absent at S twice is left to the sequential path.
__global__ __launch_bounds__(kSpecThreads) void spec_hits_kernel(BmArgs a) {
  __shared__ int32_t wave_miss[kPosPer][kBmWaves];
  const BmState& s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t n = (int32_t)s.sp_ctr[kSpN];
  for (int32_t j = blockIdx.x; j < n; j += gridDim.x) {
    const int32_t m = s.sp_m[j], nt = s.sp_ntok[j];
    const int nq = (m + kSpecThreads - 1) / kSpecThreads;  // position blocks in use (uniform)
    // position i = q * kSpecThreads + tid
    int2 v[kPosPer];
#pragma unroll
    for (int q = 0; q < kPosPer; ++q) {
      const int32_t i = q * kSpecThreads + tid;
      v[q] = int2{-1, -1};
      if (q >= nq) continue;
      bool present = false;
      if (i < m) {
        v[q] = s.sp_p0[(int64_t)j * kSpecPos + i];
        if (v[q].x >= 0) {
          present = true;
        } else {
          const int32_t f = fo_find(s, a.hashes[s.sp_h0[j] + i]);
          if (f / kSpecPos < j) {
            present = true;
            v[q].x = -(f + 2);
            s.sp_p0[(int64_t)j * kSpecPos + i].x = v[q].x;
          } else if (f != j * kSpecPos + i) {
            atomicMin(spec_bad(s), j);
          }
        }
      }
      const uint64_t mb = __ballot(i < m && !present);
      if (lane == 0)
        wave_miss[q][wave] =
            mb ? q * kSpecThreads + wave * 64 + (int32_t)__builtin_ctzll(mb) : INT_MAX;
    }
    __syncthreads();
    int32_t k = m;
#pragma unroll
    for (int q = 0; q < kPosPer; ++q)
#pragma unroll
      for (int w = 0; w < kBmWaves; ++w)
        k = q < nq && wave_miss[q][w] < k ? wave_miss[q][w] : k;
    if (tid == 0) {
      s.sp_k[j] = k;
      s.sp_take[j] = (nt + 15) / 16 - k + ((nt & 15) ? 1 : 0);
    }
#pragma unroll
    for (int q = 0; q < kPosPer; ++q) {
      const int32_t i = q * kSpecThreads + tid;
      if (i < k && v[q].x >= 0 && (v[q].x & kPinBit))
        atomicMin(&s.sp_first[v[q].x & ~kPinBit], j);
      // a page found at S past the first miss: an eviction of it by this or
      // an earlier admit would change what a later admit registers (with
      // prefix keys there is none)
      if (i >= k && i < m && v[q].x >= 0) atomicMin(&s.sp_late[v[q].x & ~kPinBit], j);
    }
    __syncthreads();  // wave_miss is rewritten for the next admit
  }
}

// 4. Per admit: the pages it pins (it is their first pinner). Then the LRU
//    window the takes may reach: each entry's page, its key's slot, and
//    whether it is a victim candidate (live at S, pinned by no admit of the
//    step), live but pinned, or dead; and the candidates per chunk of
//    kWinChunk entries.
__global__ __launch_bounds__(kWinChunk) void spec_window_kernel(BmArgs a) {
  constexpr int kWaves = kWinChunk / 64;
  __shared__ int64_t part[kWaves];
  __shared__ int32_t cnt[kWaves];
  const BmState& s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t n = (int32_t)s.sp_ctr[kSpN];
  for (int32_t j = blockIdx.x; j < n; j += gridDim.x) {
    const int32_t k = s.sp_k[j];
    int32_t c = 0;
    for (int32_t i = tid; i < k; i += kWinChunk) {
      const int32_t x = s.sp_p0[(int64_t)j * kSpecPos + i].x;
      c += x >= 0 && (x & kPinBit) && s.sp_first[x & ~kPinBit] == j;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
    if (lane == 0) cnt[wave] = c;
    __syncthreads();
    if (tid == 0) {
      int32_t t = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) t += cnt[w];
      s.sp_pinned[j] = t;
    }
    __syncthreads();  // cnt is rewritten
  }
  // the evictions all admits would need, summed by every workgroup
  int64_t mine = 0;
  for (int32_t j = tid; j < n; j += kWinChunk) mine += s.sp_take[j];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mine += __shfl_xor(mine, off);
  if (lane == 0) part[wave] = mine;
  __syncthreads();
  int64_t takes = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) takes += part[w];
  const int64_t evict = takes - s.sp_ctr[kSpF];
  const int64_t head = s.sp_ctr[kSpHead], span = s.ctr[kTail] - head;
  int64_t W = evict <= 0 ? 0 : evict + evict / 2 + 4096;
  W = W < span ? W : span;
  W = W < kSpecWin ? W : kSpecWin;
  if (blockIdx.x == 0 && tid == 0) s.sp_ctr[kSpWin] = W;
  const int64_t qm = s.Q - 1;
  for (int64_t c = blockIdx.x; c * kWinChunk < W; c += gridDim.x) {
    const int64_t w = c * kWinChunk + tid;
    uint8_t f = 0;
    if (w < W) {
      const uint64_t e = s.ring[(head + w) & qm];
      const int32_t p = (int32_t)(uint32_t)e;
      const RecHead h = rec_head(s, p);
      const bool lv = live(h, (uint32_t)(e >> 32));
      f = !lv ? 0 : (s.sp_first[p] != INT_MAX ? 2 : 1);
      s.sp_wpg[w] = p;
      s.sp_wslot[w] = h.slot;
      s.sp_wflag[w] = f;
    }
    const int32_t cw = __popcll(__ballot(f == 1));
    if (lane == 0) cnt[wave] = cw;
    __syncthreads();
    if (tid == 0) {
      int32_t t = 0;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) t += cnt[v];
      s.sp_wcnt[c] = t;
    }
    __syncthreads();  // cnt is rewritten
  }
}

// The admit owning take index t (t < T[n]): the last j with T[j] <= t, T the
// exclusive prefix sums of the admits' takes.
__device__ __forceinline__ int32_t spec_owner(const int64_t* T, int32_t n, int64_t t) {
  int32_t lo = 0, hi = n - 1;
  while (lo < hi) {
    const int32_t mid = (lo + hi + 1) >> 1;
    if (T[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// 5. Per window chunk (many CUs), after the takes' prefix sums, which every
//    workgroup computes for itself (workgroup 0 also keeps them, checks each
//    admit for OOM, and checks that the window holds the evictions wanted: if
//    it is too short, the admit that lacks one is a violation). Victim v, the
//    (v+1)-th candidate in window order, is take F + v, which belongs to the
//    admit whose prefix range holds it; a live entry pinned in the step is
//    passed by the admit owning the take index it is passed at, a violation
//    if that admit comes before its first pinner (sequentially it would have
//    evicted it). A hit is never a victim (pinned, or not in the LRU at all),
//    so only pages held past a first miss can be read after their eviction.
__global__ __launch_bounds__(kWinChunk) void spec_victims_kernel(BmArgs a) {
  constexpr int kWaves = kWinChunk / 64;
  constexpr int kOpt = kSpecOps / kWinChunk;  // consecutive admits per thread
  static_assert(kOpt * kWinChunk == kSpecOps, "admits split evenly over the threads");
  __shared__ int64_t T[kSpecOps + 1];
  __shared__ int64_t wave_tot[2][kWaves];
  __shared__ int32_t cnt[kWaves];
  const BmState& s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool lead = blockIdx.x == 0;
  const int32_t n = (int32_t)s.sp_ctr[kSpN];
  const int64_t W = s.sp_ctr[kSpWin];
  if (n == 0 || (!lead && (int64_t)blockIdx.x * kWinChunk >= W)) return;  // no chunk here
  const int64_t F = s.sp_ctr[kSpF], live0 = s.sp_ctr[kSpLive];
  // exclusive prefix sums of takes and pins, kOpt consecutive admits per thread
  int64_t tk[kOpt], pn[kOpt], st = 0, sp = 0;
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    tk[u] = j < n ? s.sp_take[j] : 0;
    pn[u] = lead && j < n ? s.sp_pinned[j] : 0;
    st += tk[u];
    sp += pn[u];
  }
  int64_t it = st, ip = sp;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t a1 = __shfl_up(it, d), a2 = __shfl_up(ip, d);
    if (lane >= d) {
      it += a1;
      ip += a2;
    }
  }
  if (lane == 63) {
    wave_tot[0][wave] = it;
    wave_tot[1][wave] = ip;
  }
  __syncthreads();
  int64_t bt = it - st, bp = ip - sp;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    bt += w < wave ? wave_tot[0][w] : 0;
    bp += w < wave ? wave_tot[1][w] : 0;
  }
#pragma unroll
  for (int u = 0; u < kOpt; ++u) {
    const int j = tid * kOpt + u;
    if (j < n) {
      T[j] = bt;
      if (lead) {
        s.sp_T[j] = bt;
        // OOM: the takes exceed the free stack left plus the evictable pages
        // left, minus the ones this admit pins
        const int64_t free_j = F - bt > 0 ? F - bt : 0;
        const int64_t ev_j = live0 - bp - (bt - F > 0 ? bt - F : 0);
        if (tk[u] > free_j + ev_j - pn[u]) atomicMin(spec_bad(s), j);
      }
    }
    bt += tk[u];
    bp += pn[u];
  }
  if (tid == kWinChunk - 1) {
    T[n] = bt;  // the last thread's running sum covers every admit
    if (lead) s.sp_T[n] = bt;
  }
  __syncthreads();
  const int64_t E = T[n] - F > 0 ? T[n] - F : 0;  // evictions wanted
  const int64_t nch = (W + kWinChunk - 1) / kWinChunk;
  // the candidates in window chunks [lo, hi), summed over the workgroup
  auto cand = [&](int64_t lo, int64_t hi) __attribute__((always_inline)) {
    int64_t v = 0;
    for (int64_t c = lo + tid; c < hi; c += kWinChunk) v += s.sp_wcnt[c];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();  // wave_tot's last readers are done
    if (lane == 0) wave_tot[0][wave] = v;
    __syncthreads();
    int64_t t = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += wave_tot[0][w];
    return t;
  };
  if (lead) {
    const int64_t ncand = cand(0, nch);
    if (tid == 0 && ncand < E) atomicMin(spec_bad(s), spec_owner(T, n, F + ncand));
  }
  int64_t pre = cand(0, (int64_t)blockIdx.x < nch ? blockIdx.x : nch);
  for (int64_t c = blockIdx.x; c < nch; c += gridDim.x) {
    const int64_t w = c * kWinChunk + tid;
    const uint8_t f = w < W ? s.sp_wflag[w] : 0;
    const uint64_t bal = __ballot(f == 1);
    if (lane == 0) cnt[wave] = __popcll(bal);
    __syncthreads();
    int64_t before = pre + __popcll(bal & ((1ull << lane) - 1ull));
#pragma unroll
    for (int v = 0; v < kWaves; ++v) before += v < wave ? cnt[v] : 0;
    if (f == 1 && before < E) {
      const int32_t p = s.sp_wpg[w];
      const int32_t u = spec_owner(T, n, F + before);
      s.sp_victim[before] = p;
      s.sp_vpos[before] = (int32_t)w;
      // a holder of p past its first miss at or after u finds it evicted;
      // when the first holder comes before u, u itself is the (safe) cut
      const int32_t lt = s.sp_late[p];
      if (lt != INT_MAX) atomicMin(spec_bad(s), lt >= u ? lt : u);
    } else if (f == 2 && before < E) {
      const int32_t u = spec_owner(T, n, F + before);
      if (u < s.sp_first[s.sp_wpg[w]]) atomicMin(spec_bad(s), u);
    }
    __syncthreads();  // cnt is rewritten
    const int64_t next = c + gridDim.x < nch ? c + gridDim.x : nch;
    pre += cand(c, next);
  }
}

// 6. The admits before the first violation, a workgroup per admit: tables,
//    refcounts, cached flags and hashes, registrations (insertion by
//    compare-and-swap at the slot found at S), results.
__global__ __launch_bounds__(kSpecThreads) void spec_commit_kernel(BmArgs a) {
  const BmState& s = a.s;
  const int32_t bad = *spec_bad(s);
  const int64_t F = s.sp_ctr[kSpF];
  int32_t reused = 0;
  for (int32_t j = blockIdx.x; j < bad; j += gridDim.x) {
    const int32_t r = s.sp_req[j], nt = s.sp_ntok[j], m = s.sp_m[j], k = s.sp_k[j];
    const int32_t np = (nt + 15) / 16;
    const bool cow = (nt & 15) != 0;
    const int64_t T = s.sp_T[j];
    for (int32_t i = threadIdx.x; i < np; i += kSpecThreads) {
      const int2 v = i < m ? s.sp_p0[(int64_t)j * kSpecPos + i] : int2{-1, -1};
      int32_t page;
      if (i < k) {
        if (v.x >= 0) {
          page = v.x & ~kPinBit;
        } else {  // the key an earlier admit w registers at its position iw
          const int32_t code = -(v.x + 2), w = code / kSpecPos, iw = code % kSpecPos;
          page = spec_take_at(s, s.sp_T[w] + iw - s.sp_k[w], F);
        }
        atomicAdd(rec_ref(s, page), 2);
      } else {
        page = spec_take_at(s, T + i - k, F);
        atomicAdd(rec_ref(s, page), (cow && i == np - 1) ? 1 : 2);
        const bool reg = i < m && v.x == -1;  // absent at S, and this is its first holder
        *rec_flag(s, page) = reg ? 1 : 0;
        if (reg) {
          const uint64_t h = a.hashes[s.sp_h0[j] + i];
          *rec_hash(s, page) = h;
          reused += tab_insert_dev(s, h, page, 2, v.y & ~kTombBit) == 1;
        }
      }
      a.tables[(int64_t)r * a.tstride + i] = page;
      if (i == np - 1) {
        if (cow)
          a.cow_src[r] = page;
        else
          a.child_last[r] = page;
      }
    }
    if (threadIdx.x == 0) {
      a.hits[r] = k;
      a.status[r] = kStOk;
      if (cow) {
        const int32_t cp = spec_take_at(s, T + np - k, F);
        atomicAdd(rec_ref(s, cp), 1);
        *rec_flag(s, cp) = 0;
        a.cow_dst[r] = a.child_last[r] = cp;
      } else {
        a.cow_src[r] = a.cow_dst[r] = -1;
        if (np == 0) a.child_last[r] = -1;
      }
    }
  }
  if (reused) atomicAdd(reinterpret_cast<unsigned long long*>(s.sp_ctr + kSpReused),
                        (unsigned long long)reused);
}

// 7. The evictions' tombstones and log, the cached pages' refcounts copied
//    into their table entries, the counters, and the scratch cleared.
__global__ __launch_bounds__(kSpecThreads) void spec_finish_kernel(BmArgs a) {
  const BmState& s = a.s;
  const int32_t bad = *spec_bad(s);
  const int64_t F = s.sp_ctr[kSpF];
  const int64_t taken = bad > 0 ? s.sp_T[bad] : 0;  // takes of the committed admits
  int64_t evicted = taken - F > 0 ? taken - F : 0;
  evicted = evicted < kSpecWin ? evicted : kSpecWin;  // (always: see spec_take_at)
  const int64_t log0 = s.ctr[kLogLen];
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < evicted;
       v += (int64_t)gridDim.x * blockDim.x) {
    *ent_page(s, s.sp_wslot[s.sp_vpos[v]]) = kTomb;
    if (log0 + v < a.evict_cap) a.evict_log[log0 + v] = s.sp_victim[v];
  }
  for (int32_t j = blockIdx.x; j < bad; j += gridDim.x) {
    const int32_t np = (s.sp_ntok[j] + 15) / 16;
    for (int32_t i = threadIdx.x; i < np; i += kSpecThreads) {
      const int32_t p = a.tables[(int64_t)s.sp_req[j] * a.tstride + i];
      const RecHead h = rec_head(s, p);
      if (h.flag & 1) *ent_ref(s, h.slot) = h.ref;
    }
  }
  if (s.sp_ctr[kSpN] > 0)  // the next step finds its scratch empty
    spec_clear_scratch(s, (int64_t)blockIdx.x * blockDim.x + threadIdx.x,
                       (int64_t)gridDim.x * blockDim.x);
  if (blockIdx.x == 0 && threadIdx.x < 64) {  // one wave: the pins of the committed admits
    int64_t pins = 0;
    for (int32_t j = threadIdx.x; j < bad; j += 64) pins += s.sp_pinned[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) pins += __shfl_xor(pins, off);
    if (threadIdx.x == 0) {
      const int32_t start = (int32_t)s.run_ctr[kRunOps];
      s.ctr[kFreeTop] = F - (taken < F ? taken : F);
      if (evicted > 0) s.ctr[kHead] = s.sp_ctr[kSpHead] + s.sp_vpos[evicted - 1] + 1;
      s.ctr[kEvictable] = s.sp_ctr[kSpLive] - pins - evicted;
      s.ctr[kTombs] += evicted - s.sp_ctr[kSpReused];
      s.ctr[kLogLen] = log0 + evicted;
      s.ctr[kSpecDone] += bad;
      s.ctr[kSpecLeft] += s.sp_ctr[kSpN] - bad;
      s.run_ctr[kRunNext] = start + bad;
    }
  }
}

// The tail kernel's group pass: the admits after the speculated ones, in
// groups, while they are valid and at most kBmThreads pages long; the step
// pass takes the ops from the first one that is not (kRunNext).
__device__ void group_pass(const BmArgs& a, Shared& sh, GroupLds& gl, GroupMeta& gm) {
  const BmState& s = a.s;
  int32_t t = (int32_t)s.run_ctr[kRunNext];  // after the run and the speculated admits
  if (s.P > kGroupMaxPages) {  // the page bitmaps do not fit in LDS
    if (threadIdx.x == 0) s.run_ctr[kRunNext] = t;
    return;
  }
  int buf = 0;
  Ctrs c;
  c.free_top = s.ctr[kFreeTop];
  c.head = s.ctr[kHead];
  c.tail = s.ctr[kTail];
  c.next_stamp = s.ctr[kNextStamp];
  c.evictable = s.ctr[kEvictable];
  c.tombs = s.ctr[kTombs];
  c.log_len = s.ctr[kLogLen];
  while (t < a.num_ops) {
    if (threadIdx.x < kGroup) {
      const int u = threadIdx.x, j = t + u;
      int32_t op = -1, n = 0, nh = -1, ok = 0;
      int64_t h0 = 0;
      if (j < a.num_ops) {
        op = a.ops[j];
        if (op >= 0 && op < a.num_requests) {
          n = a.ntok[op];
          h0 = a.hash_off[op];
          const int64_t m = a.hash_off[op + 1] - h0, np = ((int64_t)n + 15) / 16;
          nh = (n >= 0 && m == n / 16) ? (int32_t)m : -1;
          ok = nh >= 0 && np <= a.twidth && np <= kBmThreads;
        }
      }
      gm.op[u] = op;
      gm.ntok[u] = n;
      gm.nhash[u] = nh;
      gm.h0[u] = h0;
      gm.ok[u] = ok;
    }
    __syncthreads();
    int g = 0;
    while (g < kGroup && gm.ok[g]) ++g;
    g = uni(g);
    if (g == 0) break;
    t += group_admit(a, gm, g, c, sh, gl, buf);  // ends with a barrier
  }
  if (threadIdx.x == 0) {
    s.run_ctr[kRunNext] = t;
    s.ctr[kFreeTop] = c.free_top;
    s.ctr[kHead] = c.head;
    s.ctr[kEvictable] = c.evictable;
    s.ctr[kTombs] = c.tombs;
    s.ctr[kLogLen] = c.log_len;
  }
}

__device__ void step_pass(const BmArgs& a, Shared& sh, OpMeta& om, AdmitLds& al) {
  int buf = 0;
  Ctrs c;
  c.free_top = a.s.ctr[kFreeTop];
  c.head = a.s.ctr[kHead];
  c.tail = a.s.ctr[kTail];
  c.next_stamp = a.s.ctr[kNextStamp];
  c.evictable = a.s.ctr[kEvictable];
  c.tombs = a.s.ctr[kTombs];
  c.log_len = a.s.ctr[kLogLen];
  if (threadIdx.x < 2) {
    sh.first_miss[threadIdx.x] = INT_MAX;
    sh.count[threadIdx.x] = 0;
    sh.tomb_reused[threadIdx.x] = 0;
  }
  for (int i = threadIdx.x; i < kSetSize; i += kBmThreads) al.claims[i] = -1;
  uint64_t cur[kHeld] = {}, nxt[kHeld] = {};
  if (a.from_start && c.tombs > a.s.C / 4) {  // what the step's setup does otherwise
    tab_rebuild(a, c);  // ends with a barrier, after every thread read the count
    if (threadIdx.x == 0) a.s.ctr[kTombs] = 0;
  }
  // the leading run of releases (if any) was retired by the run kernels, and
  // the admits after it by the speculation and the group pass
  const int32_t start = a.from_start ? 0 : (int32_t)a.s.run_ctr[kRunNext];
  for (int32_t base = start; base < a.num_ops; base += kOpChunk) {
    const int cnt = a.num_ops - base < kOpChunk ? a.num_ops - base : kOpChunk;
    for (int t = threadIdx.x; t < cnt; t += kBmThreads) {
      const int32_t op = a.ops[base + t];
      const int32_t r = op >= 0 ? op : -(op + 1);
      int32_t n = 0, nh = -1;
      int64_t h0 = 0;
      if (r < a.num_requests) {
        n = a.ntok[r];
        if (op >= 0) {
          h0 = a.hash_off[r];
          const int64_t m = a.hash_off[r + 1] - h0;
          nh = (n >= 0 && m == n / 16) ? (int32_t)m : -1;
        }
      }
      om.op[t] = op;
      om.ntok[t] = n;
      om.nhash[t] = nh;
      om.h0[t] = h0;
    }
    __syncthreads();
    fetch_hashes(a, om, 0, cur);
    for (int t = 0; t < cnt; ++t) {
      const int par = (base + t) & 1;
      if (threadIdx.x == 0) {  // the previous op's set (its reads ended at its last barrier)
        sh.first_miss[par ^ 1] = INT_MAX;
        sh.count[par ^ 1] = 0;
        sh.tomb_reused[par ^ 1] = 0;
      }
      // the next op's page hashes are loaded while this one runs
      if (t + 1 < cnt) fetch_hashes(a, om, t + 1, nxt);
      const int32_t op = uni(om.op[t]);
      const int32_t r = op >= 0 ? op : -(op + 1);
      if (r >= a.num_requests) {
        if (threadIdx.x == 0) raise_err(a.err, MKV_DEVERR_BM);
      } else if (op >= 0) {
        admit(a, r, uni(om.ntok[t]), uni(om.nhash[t]), uni64(om.h0[t]), cur, c, sh, al, buf, par);
      } else {
        release(a, r, uni(om.ntok[t]), c, sh, buf);
      }
      for (int i = threadIdx.x; i < kSetSize; i += kBmThreads) al.claims[i] = -1;
      __syncthreads();  // the op's writes are visible to the next op
#pragma unroll
      for (int j = 0; j < kHeld; ++j) cur[j] = nxt[j];
    }
    __syncthreads();  // the staged metadata is rewritten by the next chunk
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

// The ops the release run and the speculation left, in order: admits in
// groups while they qualify, then one op at a time (a short step: every op,
// one at a time). One kernel, the two passes' LDS overlaid.
union TailLds {
  struct {
    GroupLds gl;
    GroupMeta gm;
  } g;
  struct {
    OpMeta om;
    AdmitLds al;
  } o;
};

__global__ __launch_bounds__(kBmThreads) void bm_tail_kernel(BmArgs a) {
  __shared__ Shared sh;
  __shared__ TailLds tl;
  if (!a.from_start) {
    group_pass(a, sh, tl.g.gl, tl.g.gm);
    __syncthreads();  // its counters and LDS reads are done before the step pass
  }
  step_pass(a, sh, tl.o.om, tl.o.al);
}

// Read-only lookup (mkv_hash_probe): one workgroup per request probes its page
// hashes 256 at a time; the first miss comes from an LDS minimum.
constexpr int kProbeThreads = 256;

__global__ __launch_bounds__(kProbeThreads) void probe_kernel(BmState s, const uint64_t* hashes,
                                                              const int64_t* off, int32_t* pages,
                                                              int32_t* hits, int32_t* err) {
  __shared__ int32_t first_miss;
  const int32_t r = blockIdx.x;
  const int64_t h0 = off[r], m = off[r + 1] - h0;
  if (threadIdx.x == 0) first_miss = INT_MAX;
  __syncthreads();
  if (m < 0) {
    if (threadIdx.x == 0) {
      hits[r] = 0;
      raise_err(err, MKV_DEVERR_TABLE);
    }
    return;
  }
  int32_t miss = INT_MAX;
  for (int64_t i = threadIdx.x; i < m; i += kProbeThreads) {
    const int32_t p = tab_find(s, hashes[h0 + i]).page;
    pages[h0 + i] = p;
    if (p < 0 && (int32_t)i < miss) miss = (int32_t)i;
  }
  miss = wave_min(miss);
  if ((threadIdx.x & 63) == 0 && miss != INT_MAX) atomicMin(&first_miss, miss);
  __syncthreads();
  if (threadIdx.x == 0) hits[r] = first_miss < m ? first_miss : (int32_t)m;
}

__global__ __launch_bounds__(256) void bm_init_kernel(BmState s, const int32_t* free_order) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = g; i < s.C; i += stride) {
    *ent_key(s, i) = 0;
    *reinterpret_cast<uint64_t*>(ent_page(s, i)) = (uint32_t)kEmpty;  // page -1, unused 0
  }
  for (int64_t p = g; p < s.P; p += stride) {
    *reinterpret_cast<u32x4*>(s.rec + p * kRecBytes) = u32x4{0u, 0u, 0u, 0xffffffffu};
    *reinterpret_cast<u32x4*>(s.rec + p * kRecBytes + 16) = u32x4{0u, 0u, 0u, 0u};
    s.free_list[p] = free_order ? free_order[p] : (int32_t)p;
  }
  for (int64_t q = g; q < s.Q; q += stride) s.ring[q] = 0;
  for (int64_t p = g; p < s.P; p += stride) s.last[p] = -1;
  spec_clear_scratch(s, g, stride);
  if (g < kNumCtr) s.ctr[g] = g == kFreeTop ? s.P : (g == kNextStamp ? 1 : 0);
  if (g < kRunNumCtr) s.run_ctr[g] = 0;
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
  const int64_t v[10] = {l.C,        l.Q,        l.off_ctr,  l.off_ent, l.off_rec,
                         l.off_free, l.off_ring, l.off_last, l.off_run, l.bytes};
  for (int i = 0; i < 10; ++i) out[i] = v[i];
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

namespace {

// The arguments of mkv_bm_step and its two halves, checked; MKV_OK with
// a.num_ops == 0 means there is nothing to launch.
int bm_step_args(BmArgs& a, const char* fn, void* state, int32_t num_pages, const int32_t* ops,
                 int32_t num_ops, int32_t num_requests, const uint64_t* page_hashes,
                 const int64_t* hash_offsets, const int32_t* num_tokens, int32_t* tables,
                 int64_t table_stride, int32_t table_width, int32_t* hits, int32_t* child_last,
                 int32_t* cow_src, int32_t* cow_dst, int32_t* status, int32_t* evict_log,
                 int64_t evict_log_capacity, int32_t* err) {
  a.num_ops = 0;
  MKV_REQUIRE(num_ops >= 0 && num_pages > 0 && table_width >= 0 && num_requests >= 0,
              MKV_E_INVALID, "%s: bad sizes", fn);
  if (num_ops == 0) return MKV_OK;
  MKV_REQUIRE(state && ops && hash_offsets && num_tokens && tables && hits && child_last &&
                  cow_src && cow_dst && status && err,
              MKV_E_INVALID, "%s: null pointer", fn);
  MKV_REQUIRE(evict_log || evict_log_capacity == 0, MKV_E_INVALID,
              "%s: eviction log capacity without a log", fn);
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
  a.from_start = num_ops <= kShortStepOps;
  return MKV_OK;
}

// The leading run of releases, then the speculation over the admits after it;
// nothing for a short step.
void launch_bm_begin(const BmArgs& a, hipStream_t st) {
  if (a.from_start) return;
  hipLaunchKernelGGL(step_setup_kernel, dim3(1), dim3(kBmThreads), 0, st, a);
  hipLaunchKernelGGL(run_drop_kernel, dim3(kDropGrid), dim3(kRunThreads), 0, st, a);
  hipLaunchKernelGGL(run_mark_kernel, dim3(kPassGrid), dim3(kRunThreads), 0, st, a);
  hipLaunchKernelGGL(run_push_kernel, dim3(kPassGrid + kSpecGrid), dim3(kRunThreads), 0, st, a);
  hipLaunchKernelGGL(spec_hits_kernel, dim3(kSpecGrid), dim3(kSpecThreads), 0, st, a);
  hipLaunchKernelGGL(spec_window_kernel, dim3(kSpecGrid), dim3(kWinChunk), 0, st, a);
  hipLaunchKernelGGL(spec_victims_kernel, dim3(kSpecGrid), dim3(kWinChunk), 0, st, a);
  hipLaunchKernelGGL(spec_commit_kernel, dim3(kSpecGrid), dim3(kSpecThreads), 0, st, a);
  hipLaunchKernelGGL(spec_finish_kernel, dim3(kSpecGrid), dim3(kSpecThreads), 0, st, a);
}

// The ops the speculation left, in order: admits in groups, then one at a time
// (a short step: every op, one at a time).
void launch_bm_end(const BmArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(bm_tail_kernel, dim3(1), dim3(kBmThreads), 0, st, a);
}

}  // namespace

extern "C" int mkv_bm_step(void* state, int32_t num_pages, const int32_t* ops, int32_t num_ops,
                           int32_t num_requests, const uint64_t* page_hashes,
                           const int64_t* hash_offsets, const int32_t* num_tokens,
                           int32_t* tables, int64_t table_stride, int32_t table_width,
                           int32_t* hits, int32_t* child_last, int32_t* cow_src,
                           int32_t* cow_dst, int32_t* status, int32_t* evict_log,
                           int64_t evict_log_capacity, int32_t* err, void* stream) {
  clear_error();
  BmArgs a;
  const int rc = bm_step_args(a, "mkv_bm_step", state, num_pages, ops, num_ops, num_requests,
                              page_hashes, hash_offsets, num_tokens, tables, table_stride,
                              table_width, hits, child_last, cow_src, cow_dst, status, evict_log,
                              evict_log_capacity, err);
  if (rc != MKV_OK || a.num_ops == 0) return rc;
  launch_bm_begin(a, as_stream(stream));
  launch_bm_end(a, as_stream(stream));
  return check_launch("mkv_bm_step");
}

extern "C" int mkv_bm_step_begin(void* state, int32_t num_pages, const int32_t* ops,
                                 int32_t num_ops, int32_t num_requests,
                                 const uint64_t* page_hashes, const int64_t* hash_offsets,
                                 const int32_t* num_tokens, int32_t* tables,
                                 int64_t table_stride, int32_t table_width, int32_t* hits,
                                 int32_t* child_last, int32_t* cow_src, int32_t* cow_dst,
                                 int32_t* status, int32_t* evict_log,
                                 int64_t evict_log_capacity, int32_t* err, void* stream) {
  clear_error();
  BmArgs a;
  const int rc = bm_step_args(a, "mkv_bm_step_begin", state, num_pages, ops, num_ops,
                              num_requests, page_hashes, hash_offsets, num_tokens, tables,
                              table_stride, table_width, hits, child_last, cow_src, cow_dst,
                              status, evict_log, evict_log_capacity, err);
  if (rc != MKV_OK || a.num_ops == 0) return rc;
  launch_bm_begin(a, as_stream(stream));
  return check_launch("mkv_bm_step_begin");
}

extern "C" int mkv_bm_step_end(void* state, int32_t num_pages, const int32_t* ops,
                               int32_t num_ops, int32_t num_requests,
                               const uint64_t* page_hashes, const int64_t* hash_offsets,
                               const int32_t* num_tokens, int32_t* tables, int64_t table_stride,
                               int32_t table_width, int32_t* hits, int32_t* child_last,
                               int32_t* cow_src, int32_t* cow_dst, int32_t* status,
                               int32_t* evict_log, int64_t evict_log_capacity, int32_t* err,
                               void* stream) {
  clear_error();
  BmArgs a;
  const int rc = bm_step_args(a, "mkv_bm_step_end", state, num_pages, ops, num_ops,
                              num_requests, page_hashes, hash_offsets, num_tokens, tables,
                              table_stride, table_width, hits, child_last, cow_src, cow_dst,
                              status, evict_log, evict_log_capacity, err);
  if (rc != MKV_OK || a.num_ops == 0) return rc;
  launch_bm_end(a, as_stream(stream));
  return check_launch("mkv_bm_step_end");
}

extern "C" int mkv_hash_probe(const void* state, int32_t num_pages, const uint64_t* page_hashes,
                              const int64_t* hash_offsets, int32_t num_requests, int32_t* pages,
                              int32_t* hits, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(num_pages > 0 && num_pages <= (1 << 28) && num_requests >= 0, MKV_E_INVALID,
              "mkv_hash_probe: bad sizes");
  if (num_requests == 0) return MKV_OK;
  MKV_REQUIRE(state && page_hashes && hash_offsets && pages && hits && err, MKV_E_INVALID,
              "mkv_hash_probe: null pointer");
  MKV_REQUIRE(((uintptr_t)state & 255) == 0, MKV_E_ALIGN,
              "mkv_hash_probe: state must be 256-byte aligned");
  const BmState s = bm_state(const_cast<void*>(state), num_pages);
  hipLaunchKernelGGL(probe_kernel, dim3((unsigned)num_requests), dim3(kProbeThreads), 0,
                     as_stream(stream), s, page_hashes, hash_offsets, pages, hits, err);
  return check_launch("mkv_hash_probe");
}
