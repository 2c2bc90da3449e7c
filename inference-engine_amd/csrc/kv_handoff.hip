// kv_handoff.hip — gfx950 (MI355X) kernels and C-ABI for the paged KV-cache
// handoff: direct pool-to-pool copy, fused multi-layer pack, unpack, the
// chunked host offload / restore pipelines, and a resident request queue for
// per-request direct handoffs (kv_queue). The ABI is declared in iekv.h.
//
// All three device-side moves are one kernel template, kv_move<>, that differs
// only in where a tile comes from and where it goes:
//   direct : pool[a][src_ids[i]]  ->  pool[a][dst_ids[i]]
//   pack   : pool[a][src_ids[i]]  ->  staging[i][a]
//   unpack : staging[i][a]        ->  pool[a][dst_ids[i]]
// One workgroup owns one (array a, run of up to `run` consecutive list
// entries, chunk of each tile). With one entry per run (the default) each tile
// is split into chunks of at least the chunk size (4 KiB for launches that
// write staging: one 16-byte vector per lane; 8 KiB for launches that write a
// pool, i.e. pool-to-pool copies and unpacks of tiles at least that large:
// two), one workgroup per chunk, and the workgroup reads its id pair with
// scalar loads; tiles smaller than the chunk size are grouped instead, one
// workgroup taking a block's tiles in several consecutive arrays; a run of
// several entries stages its ids in LDS. Data moves
// with wavefront-contiguous 16-byte loads and stores (a wave64 covers 1 KiB,
// a workgroup 4 KiB per access step), keeping up to `U` loads per lane in
// flight before the matching stores. The data is never interpreted: it moves
// as raw words, so every KV dtype is bit-exact.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <new>
#include <string>
#include <type_traits>
#include <vector>

#include "iekv.h"
#include "kv_plan.h"

struct iekv_pool {
  int32_t device;
  int32_t n_arrays;
  int64_t tile_bytes;
  int64_t num_blocks;
  uint64_t base;    // slab mode: array a starts at base + a * stride
  int64_t stride;
  uint64_t* table;  // table mode: device copy of the n_arrays base addresses (else null)
  int32_t align;    // largest power of two <= 16 dividing tile_bytes and every base address
  std::vector<uint64_t> arrays;   // the n_arrays base addresses (host copy)
  uint64_t lo, hi;  // the byte range the arrays span: [lowest base, highest base + array)
};

// Staging buffer of iekv_offload_static, the allocation-free offload: every
// GPU the library runs on holds its own copy from module load until the
// process ends. Host code passes kernels the address hipGetSymbolAddress
// reports for the current device, never this name (see static_staging).
static __device__ __align__(256) unsigned char scratch[IEKV_STATIC_STAGING_BYTES];

namespace {

using iekv_plan::kBlockMajor;
using iekv_plan::kDiagonal;
using iekv_plan::kMaxGrid;
using iekv_plan::kThreads;
using iekv_plan::kXcdGrouped;
using iekv_plan::MovePlan;
using iekv_plan::Place;
using iekv_plan::place_in_grid;
constexpr int kMaxRun = 64;    // block ids staged in LDS per workgroup
constexpr int64_t kMaxTileBytes = int64_t(1) << 30;

thread_local std::string g_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

// A failed HIP call returns IEKV_ERR_HIP with the runtime's message, and
// leaves HIP's last error clear: the next call's own check after its launch
// must not see this failure again.
#define IEKV_HIP(expr)                                                                   \
  do {                                                                                   \
    hipError_t err_ = (expr);                                                            \
    if (err_ != hipSuccess) {                                                            \
      (void)hipGetLastError();                                                           \
      return set_error(IEKV_ERR_HIP, "%s: %s", #expr, hipGetErrorString(err_));          \
    }                                                                                    \
  } while (0)

// Launch shape. Measured on MI355X over the five benchmark workloads (8 KiB to
// 64 KiB tiles): one tile per workgroup and streaming (non-temporal) accesses
// are best or within noise everywhere; unroll 4, 8 and 16 are within noise of
// each other, and 8 keeps the kernel at 62 VGPRs (full occupancy).
std::atomic<int> g_run{0};       // 0 = automatic
std::atomic<int> g_unroll{8};
std::atomic<int> g_nontemporal{1};
// Workgroup order (described at kv_move) of launches that write a pool (direct,
// unpack, restore): XCD-grouped block-major, so each XCD streams through its
// own eighth of the arrays. Over 11 pool paddings of the Llama-3-70B-share
// shape it averaged 6.20 TB/s (worst 5.90) against 5.88 (worst 5.00) for
// diagonal and 5.86 (worst 4.59) for array-major; on the Llama-3-8B shape all
// three are within 0.2%.
std::atomic<int> g_order{kXcdGrouped | kBlockMajor};
// Order of launches that write a staging buffer (pack, offload): array-major,
// so consecutive workgroups write consecutive staging tiles. Over 11 pool
// paddings each of the Llama-3-8B and 70B-share shapes it was faster than
// diagonal on every 70B-share padding (5.82 against 5.46 TB/s on average) and
// faster or tied on every 8B padding (5.66 against 5.62).
std::atomic<int> g_pack_order{0};
// Bytes each workgroup moves: a tile larger than this splits into a
// power-of-two number of chunks of at least this size, one workgroup each; a
// smaller one is moved together with the same block's tiles in the next
// arrays, up to this size per workgroup (iekv_plan::tile_group). This one is
// for the launches that write a staging buffer (pack, offload). Measured on
// MI355X in one process per workload, pools made anew each round and both
// sizes timed on the same pools: the pack ran 5.2-5.5% faster with 4 KiB than
// with 8 KiB on the Llama-3-8B and prefix-sharing workloads, 1.8% on the
// 70B share.
std::atomic<int> g_chunk{4096};
// The same setting for the launches that write a pool from HBM (chunk_of):
// pool-to-pool moves (copy_direct and its variants) and unpacks of a device or
// pageable-host staging image whose tiles are at least this large (unpacks
// that read pinned host memory move whole tiles). Measured the same way, two
// request streams: 8 KiB chunks moved the per-request direct copy at 6.52 /
// 6.50 / 6.41 TB/s (Llama-3-8B, prefix-sharing, 70B-share workloads) against
// 6.44 / 6.42 / 6.37 for 4 KiB, ahead in every placement, and the unpack
// 2.3% / 2.8% / 1.2% faster; whole tiles tied 8 KiB on the direct copy of the
// first two and lost on the third. The one loss: a small move issued as one
// launch (0.3 GB in about 37,000 workgroups) ran 4.7% slower than with 4 KiB
// chunks.
std::atomic<int> g_direct_chunk{8192};

// ---------------------------------------------------------------------------
// Device side
// ---------------------------------------------------------------------------

struct PoolView {
  const uint64_t* table;
  uint64_t base;
  int64_t stride;
  int64_t num_blocks;
};

PoolView view_of(const iekv_pool* p) {
  PoolView v{};
  if (p) {
    v.table = p->table;
    v.base = p->base;
    v.stride = p->stride;
    v.num_blocks = p->num_blocks;
  }
  return v;
}

__device__ __forceinline__ char* array_base(const PoolView& p, int a) {
  return reinterpret_cast<char*>(p.table ? p.table[a]
                                         : p.base + static_cast<uint64_t>(a) * p.stride);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Tile data is addressed through global (address space 1) pointers so the
// compiler emits global_load/global_store rather than FLAT accesses, which
// would also have to be waited for on the LDS counter.
template <typename T>
using gptr = __attribute__((address_space(1))) T*;

template <typename V>
__device__ __forceinline__ gptr<const V> as_global(const char* p) {
  return (gptr<const V>)(reinterpret_cast<const V*>(p));
}

template <typename V>
__device__ __forceinline__ gptr<V> as_global(char* p) {
  return (gptr<V>)(reinterpret_cast<V*>(p));
}

template <typename V, bool NT>
__device__ __forceinline__ V load_vec(gptr<const V> p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <typename V, bool NT>
__device__ __forceinline__ void store_vec(gptr<V> p, V v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Move one tile of `n` vectors from s to d. Lane t handles vectors
// t, t+256, ..., issuing U loads before the U stores that consume them.
template <typename V, int U, bool NT>
__device__ __forceinline__ void move_tile(gptr<const V> s, gptr<V> d, int n) {
  const int t = threadIdx.x;
  int v = t;
  const int full = n - (U - 1) * kThreads;  // v < full: all U vectors of the step are in range
  for (; v < full; v += U * kThreads) {
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = load_vec<V, NT>(s + v + u * kThreads);
#pragma unroll
    for (int u = 0; u < U; ++u) store_vec<V, NT>(d + v + u * kThreads, r[u]);
  }
  if (v < n) {
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (v + u * kThreads < n) r[u] = load_vec<V, NT>(s + v + u * kThreads);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (v + u * kThreads < n) store_vec<V, NT>(d + v + u * kThreads, r[u]);
  }
}

// Workgroups take (array unit, run of list entries, chunk) triples in the
// order iekv_plan::place_at describes (kv_plan.h). Every move launch has
// exactly units * runs * parts workgroups, so the kernels take the grid size
// from the plan (place_in_grid) and never read gridDim: no kernel of this
// library has hidden arguments, which keeps each launch's argument copy small.

#ifndef IEKV_UNPACK_LOAD_FIRST
#define IEKV_UNPACK_LOAD_FIRST 1
#endif

// Move chunk p of list entry `entry` of array a: from pool tile src_id (or the
// staging image of the entry) to pool tile dst_id (or the staging image).
// Ids outside their pool move nothing, so a bad id never addresses memory
// outside the pool.
template <typename V, int U, bool NT, bool SRC_POOL, bool DST_POOL, bool HOST = false>
__device__ __forceinline__ void move_entry(const PoolView& src, const PoolView& dst,
                                           const char* src_stage, char* dst_stage,
                                           int32_t src_id, int32_t dst_id, int64_t entry,
                                           int a, int p, int32_t tile_vecs, int32_t parts,
                                           int32_t n_arrays) {
  const int64_t tile_bytes = static_cast<int64_t>(tile_vecs) * sizeof(V);
  const int chunk_vecs = tile_vecs / parts;
  const int64_t chunk_offset = static_cast<int64_t>(p) * chunk_vecs * sizeof(V);
  if constexpr (IEKV_UNPACK_LOAD_FIRST && !SRC_POOL && DST_POOL && (U <= 4 || HOST)) {
    // Staging to pool: the chunk's address in the staging image does not depend
    // on the destination id, so its first vectors are loaded before the id is
    // checked and the two latencies overlap. From HBM staging only for up to 4
    // vectors per lane: with 8, the compiler kept a whole 32 KiB tile in
    // registers (240 VGPRs, 2 waves per SIMD) and whole-tile unpacks fell from
    // 6.7 to 4.2 TB/s (the default 4 KiB chunks move one vector per lane). An
    // unpack that reads pinned host memory (HOST) keeps it at any width: there
    // the lower occupancy measured faster on 32 KiB tiles (a 37 GB restore 56.7
    // against 53.7 GB/s, one 2 MiB block per call 50.4 against 43.1), the host
    // link taking fewer reads in flight.
    const gptr<const V> gs =
        as_global<V>(src_stage + (entry * n_arrays + a) * tile_bytes + chunk_offset);
    const int t = threadIdx.x;
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (t + u * kThreads < chunk_vecs) r[u] = load_vec<V, NT>(gs + t + u * kThreads);
    if (dst_id < 0 || dst_id >= dst.num_blocks) return;
    const gptr<V> gd = as_global<V>(array_base(dst, a) + dst_id * tile_bytes + chunk_offset);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (t + u * kThreads < chunk_vecs) store_vec<V, NT>(gd + t + u * kThreads, r[u]);
    if (chunk_vecs > U * kThreads)
      move_tile<V, U, NT>(gs + U * kThreads, gd + U * kThreads, chunk_vecs - U * kThreads);
    return;
  }
  const char* s;
  char* d;
  if constexpr (SRC_POOL) {
    if (src_id < 0 || src_id >= src.num_blocks) return;
    s = array_base(src, a) + src_id * tile_bytes;
  } else {
    s = src_stage + (entry * n_arrays + a) * tile_bytes;
  }
  if constexpr (DST_POOL) {
    if (dst_id < 0 || dst_id >= dst.num_blocks) return;
    d = array_base(dst, a) + dst_id * tile_bytes;
  } else {
    d = dst_stage + (entry * n_arrays + a) * tile_bytes;
  }
  move_tile<V, U, NT>(as_global<V>(s + chunk_offset), as_global<V>(d + chunk_offset),
                      chunk_vecs);
}

// Tiles smaller than a chunk: the workgroup moves tiles a0 .. a0 + group - 1
// (arrays past n_arrays excepted) of list entry `entry`, i.e. one block's
// tiles in `group` consecutive arrays. tile_vecs divides kThreads, so
// lane t always takes vector t % tile_vecs of a tile: of tile
// a0 + t / tile_vecs first, then of the tiles kThreads / tile_vecs further
// on, with up to U of them in flight.
template <typename V, int U, bool NT, bool SRC_POOL, bool DST_POOL>
__device__ __forceinline__ void move_group(const PoolView& src, const PoolView& dst,
                                           const char* src_stage, char* dst_stage,
                                           int32_t src_id, int32_t dst_id, int64_t entry,
                                           int a0, int32_t tile_vecs, int32_t group,
                                           int32_t n_arrays) {
  if constexpr (SRC_POOL) {
    if (src_id < 0 || src_id >= src.num_blocks) return;
  }
  if constexpr (DST_POOL) {
    if (dst_id < 0 || dst_id >= dst.num_blocks) return;
  }
  const int64_t tile_bytes = static_cast<int64_t>(tile_vecs) * sizeof(V);
  const int t = threadIdx.x;
  const int per_pass = kThreads / tile_vecs;
  const int64_t lane_offset = static_cast<int64_t>(t % tile_vecs) * sizeof(V);
  const int tiles = min(group, n_arrays - a0);
  auto src_of = [&](int a) -> const char* {
    if constexpr (SRC_POOL) return array_base(src, a) + src_id * tile_bytes + lane_offset;
    else return src_stage + (entry * n_arrays + a) * tile_bytes + lane_offset;
  };
  auto dst_of = [&](int a) -> char* {
    if constexpr (DST_POOL) return array_base(dst, a) + dst_id * tile_bytes + lane_offset;
    else return dst_stage + (entry * n_arrays + a) * tile_bytes + lane_offset;
  };
  for (int j = t / tile_vecs; j < tiles; j += U * per_pass) {
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j + u * per_pass < tiles)
        r[u] = load_vec<V, NT>(as_global<V>(src_of(a0 + j + u * per_pass)));
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j + u * per_pass < tiles)
        store_vec<V, NT>(as_global<V>(dst_of(a0 + j + u * per_pass)), r[u]);
  }
}

// One list entry's share of a workgroup: chunk p of its tile in array a, or,
// with group > 1, its tiles in arrays a * group .. a * group + group - 1. The
// grouped path keeps at most 4 vectors per lane in flight: each one carries
// its own source and destination address, and at 8 the kernel's register
// count would lower the occupancy of every launch it serves.
template <typename V, int U, bool NT, bool SRC_POOL, bool DST_POOL, bool HOST = false>
__device__ __forceinline__ void move_unit(const PoolView& src, const PoolView& dst,
                                          const char* src_stage, char* dst_stage,
                                          int32_t src_id, int32_t dst_id, int64_t entry,
                                          int a, int p, int32_t tile_vecs, int32_t parts,
                                          int32_t group, int32_t n_arrays) {
  if (group > 1)
    move_group<V, (U < 4 ? U : 4), NT, SRC_POOL, DST_POOL>(
        src, dst, src_stage, dst_stage, src_id, dst_id, entry, a * group, tile_vecs, group,
        n_arrays);
  else
    move_entry<V, U, NT, SRC_POOL, DST_POOL, HOST>(src, dst, src_stage, dst_stage, src_id, dst_id,
                                             entry, a, p, tile_vecs, parts, n_arrays);
}

// Ids in device memory. A one-block workgroup reads its id pair with uniform
// (scalar) loads: staging it in LDS would add a store, a barrier and a load
// before the first data access of a workgroup that lives for a single chunk.
// A run of several blocks stages its slice of the src -> dst id map in LDS.
template <typename V, int U, bool NT, bool SRC_POOL, bool DST_POOL, bool HOST>
__global__ void __launch_bounds__(kThreads)
kv_move(PoolView src, PoolView dst, const char* __restrict__ src_stage,
        char* __restrict__ dst_stage, const int32_t* __restrict__ src_ids,
        const int32_t* __restrict__ dst_ids, int32_t tile_vecs, int32_t n_blocks,
        int32_t n_arrays, int32_t run, int32_t runs, int32_t parts, int32_t group,
        int32_t order) {
  __shared__ int32_t s_src[kMaxRun];
  __shared__ int32_t s_dst[kMaxRun];
  const Place pl = place_in_grid(blockIdx.x, (n_arrays + group - 1) / group, runs, parts, order);
  const int first = pl.r * run;
  if (run == 1) {
    move_unit<V, U, NT, SRC_POOL, DST_POOL, HOST>(
        src, dst, src_stage, dst_stage, SRC_POOL ? src_ids[first] : 0,
        DST_POOL ? dst_ids[first] : 0, first, pl.a, pl.p, tile_vecs, parts, group, n_arrays);
    return;
  }
  const int count = min(run, n_blocks - first);
  const int t = threadIdx.x;
  if (t < count) {
    if constexpr (SRC_POOL) s_src[t] = src_ids[first + t];
    if constexpr (DST_POOL) s_dst[t] = dst_ids[first + t];
  }
  __syncthreads();
  for (int j = 0; j < count; ++j)
    move_unit<V, U, NT, SRC_POOL, DST_POOL, HOST>(
        src, dst, src_stage, dst_stage, SRC_POOL ? s_src[j] : 0, DST_POOL ? s_dst[j] : 0,
        first + j, pl.a, pl.p, tile_vecs, parts, group, n_arrays);
}

// Ids carried in the launch's own kernel arguments: source ids at ids[i],
// destination ids at ids[dst_off + i], for list entries id_base + i. One block
// per workgroup; each workgroup reads its id pair with scalar loads from the
// kernel-argument segment, so no id buffer or upload is needed.
// The runtime copies a launch's whole argument segment for every launch, and
// on slower hosts each KiB of it adds 0.5-0.8 us to the launch's host cost,
// so the id block comes in two sizes: kSmallIdWords words for short lists (a
// small workload's per-request tables) and the full 2 * IEKV_INLINE_IDS.
template <int W>
struct InlineIds {
  int32_t v[W];
};
constexpr int kSmallIdWords = 64;
constexpr int kIdWords = 2 * IEKV_INLINE_IDS;

template <typename V, int U, bool NT, bool SRC_POOL, bool DST_POOL, bool HOST, int W>
__global__ void __launch_bounds__(kThreads)
kv_move_inline(PoolView src, PoolView dst, const char* __restrict__ src_stage,
               char* __restrict__ dst_stage, InlineIds<W> ids, int32_t id_base, int32_t dst_off,
               int32_t tile_vecs, int32_t n_arrays, int32_t runs, int32_t parts,
               int32_t group, int32_t order) {
  const Place pl = place_in_grid(blockIdx.x, (n_arrays + group - 1) / group, runs, parts, order);
  const int i = id_base + pl.r;
  move_unit<V, U, NT, SRC_POOL, DST_POOL, HOST>(
      src, dst, src_stage, dst_stage, SRC_POOL ? ids.v[i] : 0, DST_POOL ? ids.v[dst_off + i] : 0,
      i, pl.a, pl.p, tile_vecs, parts, group, n_arrays);
}

// Scattered host images moved directly, in either direction: list entry i's
// image ([2L][T] bytes, device-visible pinned host memory) starts at
// images.addr[i]. A restore (DST_POOL) moves it onto block ids[i]; an offload
// (SRC_POOL) packs block ids[i] into it. With ids null the ids are
// images.ids[i]. The addresses, and host-side ids, ride in the kernel
// arguments. move_unit addresses entry i's image at stage + i * 2L * T, so
// shifting the base back by that much points it at images.addr[i].
struct InlineImages {
  uint64_t addr[IEKV_INLINE_IMAGES];
  int32_t ids[IEKV_INLINE_IMAGES];  // block ids, when they come from host memory
};

template <typename V, int U, bool NT, bool SRC_POOL, bool DST_POOL, bool HOST>
__global__ void __launch_bounds__(kThreads)
kv_move_images(PoolView src, PoolView dst, const char* __restrict__ /*src_stage*/,
               char* __restrict__ /*dst_stage*/, InlineImages images,
               const int32_t* __restrict__ ids, int32_t tile_vecs, int32_t n_arrays,
               int32_t runs, int32_t parts, int32_t group, int32_t order) {
  static_assert(SRC_POOL != DST_POOL, "images are packed from, or restored into, a pool");
  const Place pl = place_in_grid(blockIdx.x, (n_arrays + group - 1) / group, runs, parts, order);
  const int i = pl.r;
  const uint64_t image_bytes = static_cast<uint64_t>(n_arrays) * tile_vecs * sizeof(V);
  char* stage = reinterpret_cast<char*>(images.addr[i] - i * image_bytes);
  const int32_t id = ids ? ids[i] : images.ids[i];
  move_unit<V, U, NT, SRC_POOL, DST_POOL, HOST>(src, dst, stage, stage, SRC_POOL ? id : 0,
                                          DST_POOL ? id : 0, i, pl.a, pl.p, tile_vecs, parts,
                                          group, n_arrays);
}

// Row kernels on either side of the handoff. A pool row is one token's
// H x D values of one array (tile_bytes / block_size bytes); row r of array a
// lives at base(a) + r * row_bytes, i.e. slot r of the reference's [N*bs, H, D]
// array. `lanes` lanes (a power of two, at most a wave) move one row with
// lane-contiguous vectors, so a workgroup moves kThreads / lanes consecutive
// rows of one array, and short rows do not leave most of a wave idle; a lane
// keeps up to U vectors of its row in flight before storing them.
// A launch covers `chunks` groups of rows in each of its arrays, workgroup w
// taking group w % chunks of array w / chunks; with `xcd`, position w is
// XCD-grouped (kv_plan.h), so each of the 8 XCDs walks its own contiguous
// share of arrays and rows. The scatter takes the XCD grouping from the order
// of pool-writing launches, the gather from that of staging-writing ones.
// Measured on MI355X, one launch per request, every layer or array at once
// (GB/s, one box):
//   Llama-3-8B shape (2 KiB rows): scatter 5,351 plain order -> 6,407 grouped,
//     with non-temporal loads and stores (6,188 with ordinary stores); gather
//     6,050 plain -> 5,698 grouped, so the gather stays in plain order;
//   70B share, fp8 (1 KiB rows): scatter 5,677 plain, 5,566 grouped;
//   one tensor-parallel rank of the 8B shape (256 B rows): scatter 4,880 plain,
//     4,480 grouped, 5,091 with ordinary accesses.
// One row per lane group beat two to eight in flight on both shapes.
constexpr int kWave = 64;
constexpr int kRowU = 4;  // vectors per lane in flight: a 4 KiB row in one step
// Stores of the scatter are non-temporal when the launch setting asks for
// non-temporal accesses (the gather's always are then).
#ifndef IEKV_SCATTER_NT_STORES
#define IEKV_SCATTER_NT_STORES 1
#endif

struct RowShape {
  int32_t row_vecs;  // vectors per row
  int32_t lanes;     // lanes per row (a power of two dividing kWave)
  int32_t chunks;    // groups of kThreads / lanes rows per array
  int32_t xcd;       // 1: XCD-grouped workgroup positions
  int32_t groups;    // workgroups in the launch (chunks * arrays; read instead of gridDim)
};

// The (array index, first row) of this workgroup.
__device__ __forceinline__ void row_place(const RowShape& sh, int* array, int64_t* first) {
  const int w = sh.xcd ? iekv_plan::xcd_grouped(blockIdx.x, sh.groups) : blockIdx.x;
  *array = w / sh.chunks;
  *first = static_cast<int64_t>(w % sh.chunks) * (kThreads / sh.lanes);
}

// Row `row` (< n) of this workgroup's share: addr(row, &src, &dst) gives its
// addresses, or false to skip it (an id outside the pool). With WAVE_ROW (a
// row spans the whole wave) the row index is made wave-uniform, so the id the
// row's addresses depend on (a slot, a table entry) is read with one scalar load
// instead of a vector load by all 64 lanes.
template <bool WAVE_ROW, typename V, bool NTL, bool NTS, typename RowAddr>
__device__ __forceinline__ void move_row_as(int64_t first, int32_t n, const RowShape& sh,
                                            RowAddr addr) {
  const int lanes = WAVE_ROW ? kWave : sh.lanes;
  const int lane = threadIdx.x & (lanes - 1);
  const int64_t row =
      first + (WAVE_ROW ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave)
                        : static_cast<int>(threadIdx.x) / lanes);
  gptr<const V> s;
  gptr<V> d;
  if (row >= n || !addr(row, &s, &d)) return;
  for (int e = lane; e < sh.row_vecs; e += kRowU * lanes) {
    V v[kRowU];
#pragma unroll
    for (int u = 0; u < kRowU; ++u)
      if (e + u * lanes < sh.row_vecs) v[u] = load_vec<V, NTL>(s + e + u * lanes);
#pragma unroll
    for (int u = 0; u < kRowU; ++u)
      if (e + u * lanes < sh.row_vecs) store_vec<V, NTS>(d + e + u * lanes, v[u]);
  }
}

// The gather reads its table entry with a scalar load when a row spans the
// wave; the scatter keeps the vector load of its slot. Measured in alternating
// processes on MI355X (two rounds each): the scalar load took the gather from
// 6,388 / 6,385 to 6,664 / 6,713 GB/s on the 70B-shape share's 1 KiB rows and
// from 6,096 / 6,100 to 6,148 / 6,151 on the 8B shape's 2 KiB rows; the scatter
// read 5,322 / 5,342 with it against 5,592 / 6,156 without on the 1 KiB rows,
// and tied on the 2 KiB rows.
#ifndef IEKV_GATHER_UNIFORM_IDS
#define IEKV_GATHER_UNIFORM_IDS 1
#endif

template <bool UNIFORM_IDS, typename V, bool NTL, bool NTS, typename RowAddr>
__device__ __forceinline__ void move_row(int64_t first, int32_t n, const RowShape& sh,
                                         RowAddr addr) {
  if (UNIFORM_IDS && sh.lanes == kWave)
    move_row_as<true, V, NTL, NTS>(first, n, sh, addr);
  else
    move_row_as<false, V, NTL, NTS>(first, n, sh, addr);
}

// The scatter loads a row's first vectors before it reads the row's slot, so
// the two memory latencies overlap instead of adding up. Measured in five
// rounds of alternating processes on MI355X: the 70B-shape share's write_kv
// (1 KiB rows) read 6,126 / 5,376 / 6,302 / 6,292 / 6,293 GB/s against
// 5,475 / 5,526 / 5,473 / 5,568 / 5,481 with the slot read first; on the 8B
// shape both orders fell into the same two placement modes (5.2-5.4 and
// 6.3-6.4 TB/s). Reading the slot with a scalar load as well measured 5,290 /
// 5,337 on the 1 KiB rows, so it stays a vector load.
#ifndef IEKV_SCATTER_LOAD_FIRST
#define IEKV_SCATTER_LOAD_FIRST 1
#endif

// A row whose source address is known before its destination: the row's first
// vectors are loaded before the destination id is read. src_of(row) gives the
// source, dst_of(row, &d) the destination or false to skip the row.
template <bool WAVE_ROW, typename V, bool NTL, bool NTS, typename Src, typename Dst>
__device__ __forceinline__ void move_row_load_first(int64_t first, int32_t n,
                                                    const RowShape& sh, Src src_of, Dst dst_of) {
  const int lanes = WAVE_ROW ? kWave : sh.lanes;
  const int lane = threadIdx.x & (lanes - 1);
  const int64_t row =
      first + (WAVE_ROW ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave)
                        : static_cast<int>(threadIdx.x) / lanes);
  if (row >= n) return;
  const gptr<const V> s = src_of(row);
  V v[kRowU];
  int e = lane;
#pragma unroll
  for (int u = 0; u < kRowU; ++u)
    if (e + u * lanes < sh.row_vecs) v[u] = load_vec<V, NTL>(s + e + u * lanes);
  gptr<V> d;
  if (!dst_of(row, &d)) return;
  while (true) {
#pragma unroll
    for (int u = 0; u < kRowU; ++u)
      if (e + u * lanes < sh.row_vecs) store_vec<V, NTS>(d + e + u * lanes, v[u]);
    e += kRowU * lanes;
    if (e >= sh.row_vecs) break;
#pragma unroll
    for (int u = 0; u < kRowU; ++u)
      if (e + u * lanes < sh.row_vecs) v[u] = load_vec<V, NTL>(s + e + u * lanes);
  }
}

// write_kv over layers: row i of layer l of k (and of v), at
// k + l * layer_stride + i * row_bytes, lands in row slots[i] of K array
// first_layer + l (and of V array layers + first_layer + l). Array index y of
// the launch is K of layer y for y < n_layers, then V.
template <typename V, bool NTL, bool NTS>
__global__ void __launch_bounds__(kThreads)
kv_scatter_rows(PoolView pool, int32_t layers, int32_t first_layer, int32_t n_layers,
                const char* __restrict__ k, const char* __restrict__ v, int64_t layer_stride,
                const int64_t* __restrict__ slots, int32_t n, RowShape sh, int64_t pool_rows) {
  int y;
  int64_t first;
  row_place(sh, &y, &first);
  const bool is_v = y >= n_layers;
  const int l = is_v ? y - n_layers : y;
  const int64_t row_bytes = static_cast<int64_t>(sh.row_vecs) * sizeof(V);
  const char* src = (is_v ? v : k) + l * layer_stride;
  char* dst = array_base(pool, (is_v ? layers : 0) + first_layer + l);
  if (IEKV_SCATTER_LOAD_FIRST) {
    auto src_of = [&](int64_t i) { return as_global<V>(src + i * row_bytes); };
    auto dst_of = [&](int64_t i, gptr<V>* d) {
      const int64_t slot = slots[i];
      if (slot < 0 || slot >= pool_rows) return false;  // never address outside the pool
      *d = as_global<V>(dst + slot * row_bytes);
      return true;
    };
    move_row_load_first<false, V, NTL, NTS>(first, n, sh, src_of, dst_of);
    return;
  }
  move_row<false, V, NTL, NTS>(
      first, n, sh, [&](int64_t i, gptr<const V>* s, gptr<V>* d) {
        const int64_t slot = slots[i];
        if (slot < 0 || slot >= pool_rows) return false;  // never address outside the pool
        *s = as_global<V>(src + i * row_bytes);
        *d = as_global<V>(dst + slot * row_bytes);
        return true;
      });
}

// gather_context over arrays: out row j (j < n) of array first_array + y, at
// out + y * out_stride + j * row_bytes, is row table[j / bs] * bs + j % bs of
// that array.
template <typename V, bool NTL, bool NTS>
__global__ void __launch_bounds__(kThreads)
kv_gather_rows(PoolView pool, int32_t first_array, const int32_t* __restrict__ table,
               int32_t bs, char* __restrict__ out, int64_t out_stride, int32_t n,
               RowShape sh) {
  int y;
  int64_t first;
  row_place(sh, &y, &first);
  const int64_t row_bytes = static_cast<int64_t>(sh.row_vecs) * sizeof(V);
  const char* base = array_base(pool, first_array + y);
  char* dst = out + y * out_stride;
  move_row<IEKV_GATHER_UNIFORM_IDS != 0, V, NTL, NTS>(
      first, n, sh, [&](int64_t j, gptr<const V>* s, gptr<V>* d) {
    const int32_t block = table[j / bs];
    if (block < 0 || block >= pool.num_blocks) return false;
    *s = as_global<V>(base + (static_cast<int64_t>(block) * bs + j % bs) * row_bytes);
    *d = as_global<V>(dst + j * row_bytes);
    return true;
  });
}

// Block-id checks of iekv_check_ids, three launches in stream order: clear the
// destination bitmap (one bit per destination block) and the status word; mark
// every destination id in the bitmap (the atomic's old word tells whether the
// id came earlier); probe every source id (against the bitmap when both lists
// index one pool). A bit of *status is set only when a check fails, so a valid
// list costs one id load and, for a destination, one bitmap atomic per id.
__global__ void __launch_bounds__(kThreads)
ids_clear(uint32_t* __restrict__ bitmap, int64_t words, int32_t* __restrict__ status,
          int32_t workgroups) {
  const int64_t stride = static_cast<int64_t>(workgroups) * kThreads;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; w < words;
       w += stride)
    bitmap[w] = 0u;
  if (blockIdx.x == 0 && threadIdx.x == 0) *status = 0;
}

__global__ void __launch_bounds__(kThreads)
ids_mark(const int32_t* __restrict__ ids, int32_t n, int64_t num_blocks,
         uint32_t* __restrict__ bitmap, int32_t* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int32_t id = ids[i];
  if (id < 0 || id >= num_blocks) {
    atomicOr(status, IEKV_IDS_DST_RANGE);
    return;
  }
  const uint32_t bit = 1u << (id & 31);
  if (atomicOr(&bitmap[id >> 5], bit) & bit) atomicOr(status, IEKV_IDS_DST_REPEATED);
}

__global__ void __launch_bounds__(kThreads)
ids_probe(const int32_t* __restrict__ ids, int32_t n, int64_t num_blocks,
          const uint32_t* __restrict__ bitmap, int32_t* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int32_t id = ids[i];
  if (id < 0 || id >= num_blocks) {
    atomicOr(status, IEKV_IDS_SRC_RANGE);
    return;
  }
  if (bitmap && (bitmap[id >> 5] >> (id & 31)) & 1u) atomicOr(status, IEKV_IDS_OVERLAP);
}

// The launch floor (iekv_noop): a kernel that does nothing, so its duration is
// the cost of dispatching, running and retiring its workgroups alone.
__global__ void __launch_bounds__(kThreads) kv_noop() {}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Per-thread launch timing: while a session is open, every kernel launch of the
// library (kv_move and the row kernels) is dispatched with hipExtLaunchKernelGGL
// carrying a start/stop event pair, so the timestamps come from the dispatch
// packet itself and no marker packets are added to the queue between launches.
struct Profiler {
  bool on = false;
  int device = -1;
  size_t used = 0;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events;

  void release() {
    for (auto& e : events) {
      (void)hipEventDestroy(e.first);
      (void)hipEventDestroy(e.second);
    }
    events.clear();
  }
  ~Profiler() { release(); }
};
thread_local Profiler g_profiler;

using MoveKernel = void (*)(PoolView, PoolView, const char*, char*, const int32_t*,
                            const int32_t*, int32_t, int32_t, int32_t, int32_t, int32_t,
                            int32_t, int32_t, int32_t);
using ImagesKernel = void (*)(PoolView, PoolView, const char*, char*, InlineImages,
                              const int32_t*, int32_t, int32_t, int32_t, int32_t, int32_t,
                              int32_t);
template <int W>
using InlineKernel = void (*)(PoolView, PoolView, const char*, char*, InlineIds<W>, int32_t,
                              int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t);

// Kernel for vectors of the widest width the alignment allows, keeping up to
// `unroll` of them in flight per lane; `lane_vecs` (vectors per lane per
// chunk) caps the unroll so small chunks do not carry dead predicated slots.
// IEKV_EXTRA holds template arguments after HOST (the inline kernels' id-block
// size W), empty for the other kernels.
#define IEKV_EXTRA
#define IEKV_PICK(KERNEL)                                                                       \
  if (align >= 16) {                                                                            \
    *vec_bytes = 16;                                                                            \
    const int u = std::min(unroll, lane_vecs);                                                  \
    if (nt) {                                                                                   \
      if (u >= 16) return KERNEL<u32x4, 16, true, SP, DP, HP IEKV_EXTRA>;                       \
      if (u >= 8) return KERNEL<u32x4, 8, true, SP, DP, HP IEKV_EXTRA>;                         \
      if (u >= 4) return KERNEL<u32x4, 4, true, SP, DP, HP IEKV_EXTRA>;                         \
      if (u >= 2) return KERNEL<u32x4, 2, true, SP, DP, HP IEKV_EXTRA>;                         \
      return KERNEL<u32x4, 1, true, SP, DP, HP IEKV_EXTRA>;                                     \
    }                                                                                           \
    if (u >= 16) return KERNEL<u32x4, 16, false, SP, DP, HP IEKV_EXTRA>;                        \
    if (u >= 8) return KERNEL<u32x4, 8, false, SP, DP, HP IEKV_EXTRA>;                          \
    if (u >= 4) return KERNEL<u32x4, 4, false, SP, DP, HP IEKV_EXTRA>;                          \
    if (u >= 2) return KERNEL<u32x4, 2, false, SP, DP, HP IEKV_EXTRA>;                          \
    return KERNEL<u32x4, 1, false, SP, DP, HP IEKV_EXTRA>;                                      \
  }                                                                                             \
  if (align >= 8) { *vec_bytes = 8; return KERNEL<u32x2, 4, false, SP, DP, HP IEKV_EXTRA>; }    \
  if (align >= 4) { *vec_bytes = 4; return KERNEL<uint32_t, 4, false, SP, DP, HP IEKV_EXTRA>; } \
  if (align >= 2) { *vec_bytes = 2; return KERNEL<uint16_t, 4, false, SP, DP, HP IEKV_EXTRA>; } \
  *vec_bytes = 1;                                                                               \
  return KERNEL<uint8_t, 4, false, SP, DP, HP IEKV_EXTRA>;

template <bool SP, bool DP, bool HP>
MoveKernel pick_kernel_as(int align, int unroll, int lane_vecs, bool nt, int* vec_bytes) {
  IEKV_PICK(kv_move)
}

template <bool SP, bool DP, bool HP>
ImagesKernel pick_images_kernel_as(int align, int unroll, int lane_vecs, bool nt,
                                   int* vec_bytes) {
  IEKV_PICK(kv_move_images)
}
#undef IEKV_EXTRA
#define IEKV_EXTRA , W
template <bool SP, bool DP, bool HP, int W>
InlineKernel<W> pick_inline_kernel_as(int align, int unroll, int lane_vecs, bool nt,
                                      int* vec_bytes) {
  IEKV_PICK(kv_move_inline)
}
#undef IEKV_EXTRA
#define IEKV_EXTRA
#undef IEKV_PICK

// The kernels of a move; `host`: an unpack that reads pinned host memory (move_entry's
// HOST variant). Only unpacks have one.
#define IEKV_PICK_HOST(NAME)                                                                    \
  if constexpr (!SP && DP) {                                                                    \
    if (host) return NAME##_as<SP, DP, true IEKV_EXTRA>(align, unroll, lane_vecs, nt, vec_bytes); \
  }                                                                                             \
  return NAME##_as<SP, DP, false IEKV_EXTRA>(align, unroll, lane_vecs, nt, vec_bytes);

template <bool SP, bool DP>
MoveKernel pick_kernel(int align, int unroll, int lane_vecs, bool nt, int* vec_bytes,
                       bool host = false) {
  IEKV_PICK_HOST(pick_kernel)
}
template <bool SP, bool DP>
ImagesKernel pick_images_kernel(int align, int unroll, int lane_vecs, bool nt, int* vec_bytes,
                                bool host = false) {
  IEKV_PICK_HOST(pick_images_kernel)
}
#undef IEKV_EXTRA
#define IEKV_EXTRA , W
template <bool SP, bool DP, int W>
InlineKernel<W> pick_inline_kernel(int align, int unroll, int lane_vecs, bool nt,
                                   int* vec_bytes, bool host = false) {
  IEKV_PICK_HOST(pick_inline_kernel)
}
#undef IEKV_EXTRA
#undef IEKV_PICK_HOST

int align_of_ptr(uint64_t p) {
  int a = 16;
  while (a > 1 && (p % a)) a >>= 1;
  return a;
}

// Makes `device` current for the lifetime of the guard and restores the
// caller's device afterwards.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) : device_(device) {
    err_ = hipGetDevice(&prev_);
    if (err_ == hipSuccess && prev_ != device) err_ = hipSetDevice(device);
    if (err_ != hipSuccess) (void)hipGetLastError();   // reported through fail()
    switched_ = err_ == hipSuccess && prev_ != device;
  }
  ~DeviceGuard() {
    if (switched_) (void)hipSetDevice(prev_);
  }
  bool ok() const { return err_ == hipSuccess; }
  // The error a caller returns when ok() is false: IEKV_ERR_HIP with the runtime's message.
  int fail() const {
    return set_error(IEKV_ERR_HIP, "cannot make device %d current: %s", device_,
                     hipGetErrorString(err_));
  }

 private:
  int device_;
  int prev_ = 0;
  hipError_t err_ = hipSuccess;
  bool switched_ = false;
};

// Whether a launch uses non-temporal loads and stores: the setting, or `nt` (0 or
// 1) when a launch chooses for itself (host_write_nontemporal).
bool nontemporal(int32_t nt) { return nt >= 0 ? nt != 0 : g_nontemporal.load() != 0; }

// Chunk size of a launch under the current settings: a pool-to-pool move takes
// the pool-writing chunk; an unpack takes it when its tiles are at least that
// large (split into pool-writing chunks), else the staging chunk, so small tiles
// stay grouped as in the pack (grouping tiles of 2-4 KiB to 8 KiB per workgroup
// slowed the unpack of the tensor-parallel shares by 1.2-3.4%); a launch that
// writes a staging image takes the staging chunk.
int32_t chunk_of(bool pool_reading, bool pool_writing, int64_t tile_bytes) {
  return iekv_plan::launch_chunk(pool_reading, pool_writing, tile_bytes, g_chunk.load(),
                                 g_direct_chunk.load());
}

// The launch shape of one move under the current settings (kv_plan.h), with
// chunk_of's chunk size; `chunk` >= 0 sets this launch's chunk size instead
// (host_read_chunk for moves that read pinned host memory).
int plan_move(int32_t n_blocks, int64_t tile_bytes, int32_t n_arrays, int align,
              bool pool_reading, bool pool_writing, bool single_blocks, MovePlan* pl,
              int32_t chunk = -1) {
  iekv_plan::Settings settings;
  settings.run = g_run.load();
  settings.chunk_bytes = chunk >= 0 ? chunk : chunk_of(pool_reading, pool_writing, tile_bytes);
  settings.order = g_order.load();
  settings.pack_order = g_pack_order.load();
  switch (iekv_plan::plan_move(n_blocks, tile_bytes, n_arrays, align, pool_writing,
                               single_blocks, settings, pl)) {
    case iekv_plan::kTileTooLarge:
      return set_error(IEKV_ERR_INVALID, "tile of %lld bytes is too large",
                       static_cast<long long>(tile_bytes));
    case iekv_plan::kTooManyArrays:
      return set_error(IEKV_ERR_INVALID, "%d arrays exceed the grid limit", n_arrays);
    default:
      return IEKV_OK;
  }
}

// One dispatch; while a timing session is open it carries a start/stop event
// pair in its own packet.
template <typename Kernel, typename... Args>
int dispatch(Kernel kernel, dim3 grid, hipStream_t stream, Args... args) {
  Profiler& prof = g_profiler;
  if (prof.on && prof.used < prof.events.size()) {
    auto& ev = prof.events[prof.used++];
    hipExtLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, ev.first, ev.second, 0,
                          args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, args...);
  }
  IEKV_HIP(hipGetLastError());
  return IEKV_OK;
}

template <bool SP, bool DP>
int launch_move(const iekv_pool* sp, const iekv_pool* dp, const char* src_stage, char* dst_stage,
                const int32_t* src_ids, const int32_t* dst_ids, int32_t n_blocks,
                int64_t tile_bytes, int32_t n_arrays, int align, hipStream_t stream,
                int32_t chunk = -1, int32_t nt = -1, bool host = false) {
  if (n_blocks == 0) return IEKV_OK;
  MovePlan pl;
  int rc;
  if ((rc = plan_move(n_blocks, tile_bytes, n_arrays, align, SP, DP, false, &pl, chunk)))
    return rc;
  MoveKernel k = pick_kernel<SP, DP>(align, g_unroll.load(), pl.lane_vecs, nontemporal(nt),
                                     &pl.vec, host);
  const int64_t block_image = tile_bytes * n_arrays;
  for (int64_t r0 = 0; r0 < pl.total_runs; r0 += pl.runs_per_launch) {
    const int64_t first = r0 * pl.run;
    const int32_t cnt = static_cast<int32_t>(
        std::min<int64_t>(pl.runs_per_launch * pl.run, n_blocks - first));
    const int32_t runs = static_cast<int32_t>((cnt + pl.run - 1) / pl.run);
    const uint32_t grid = iekv_plan::launch_workgroups(pl, runs);
    if ((rc = dispatch(k, grid, stream, view_of(sp), view_of(dp),
                       SP ? nullptr : src_stage + first * block_image,
                       DP ? nullptr : dst_stage + first * block_image,
                       SP ? src_ids + first : nullptr, DP ? dst_ids + first : nullptr,
                       pl.tile_vecs, cnt, n_arrays, pl.run, runs, pl.parts, pl.group,
                       pl.order)))
      return rc;
  }
  return IEKV_OK;
}

// The same move with its ids in the kernel arguments (n_blocks <=
// IEKV_INLINE_IDS): src ids at ids.v[i], dst ids at ids.v[dst_off + i].
template <bool SP, bool DP, int W>
int launch_move_inline(const iekv_pool* sp, const iekv_pool* dp, const char* src_stage,
                       char* dst_stage, const InlineIds<W>& ids, int32_t dst_off, int32_t n_blocks,
                       int64_t tile_bytes, int32_t n_arrays, int align, hipStream_t stream,
                       int32_t chunk = -1, int32_t nt = -1, bool host = false) {
  if (n_blocks == 0) return IEKV_OK;
  MovePlan pl;
  int rc;
  if ((rc = plan_move(n_blocks, tile_bytes, n_arrays, align, SP, DP, true, &pl, chunk)))
    return rc;
  InlineKernel<W> k = pick_inline_kernel<SP, DP, W>(align, g_unroll.load(), pl.lane_vecs,
                                                    nontemporal(nt), &pl.vec, host);
  for (int64_t r0 = 0; r0 < pl.total_runs; r0 += pl.runs_per_launch) {
    const int32_t runs = static_cast<int32_t>(std::min<int64_t>(pl.runs_per_launch,
                                                                pl.total_runs - r0));
    const uint32_t grid = iekv_plan::launch_workgroups(pl, runs);
    if ((rc = dispatch(k, grid, stream, view_of(sp), view_of(dp), src_stage, dst_stage, ids,
                       static_cast<int32_t>(r0), dst_off, pl.tile_vecs, n_arrays, runs, pl.parts,
                       pl.group, pl.order)))
      return rc;
  }
  return IEKV_OK;
}

// The scattered-image restore in one launch (n_blocks <= IEKV_INLINE_IMAGES).
template <bool SP, bool DP>
int launch_images(const iekv_pool* pool, const InlineImages& images, const int32_t* ids,
                  int32_t n_blocks, hipStream_t stream, int32_t chunk = -1,
                  int32_t nt = -1, bool host = false) {
  static_assert(SP != DP, "a pack or an unpack");
  int align = pool->align;
  for (int32_t i = 0; i < n_blocks; ++i) align = std::min(align, align_of_ptr(images.addr[i]));
  MovePlan pl;
  int rc;
  if ((rc = plan_move(n_blocks, pool->tile_bytes, pool->n_arrays, align, SP, DP, true, &pl,
                      chunk)))
    return rc;
  // At most IEKV_HOST_DIRECT_MAX_BYTES in chunks of at least 64 bytes: one launch holds them.
  if (pl.runs_per_launch < n_blocks)
    return set_error(IEKV_ERR_INVALID, "%d images do not fit one launch", n_blocks);
  ImagesKernel k = pick_images_kernel<SP, DP>(align, g_unroll.load(), pl.lane_vecs,
                                              nontemporal(nt), &pl.vec, host);
  const uint32_t grid = iekv_plan::launch_workgroups(pl, n_blocks);
  return dispatch(k, grid, stream, SP ? view_of(pool) : PoolView{},
                  DP ? view_of(pool) : PoolView{}, nullptr, nullptr, images, ids, pl.tile_vecs,
                  pool->n_arrays, n_blocks, pl.parts, pl.group, pl.order);
}

// The shape of a row launch over n rows in each of n_arrays arrays: lanes per
// row (the smallest power of two with a vector of the row for every lane, at
// most a wave), row groups per array, and the workgroup order. False when the
// launch would exceed the dispatch limit.
bool row_shape(int64_t row_bytes, int vec_bytes, int64_t n, int32_t n_arrays, bool xcd,
               RowShape* sh, uint32_t* grid) {
  sh->row_vecs = static_cast<int32_t>(row_bytes / vec_bytes);
  sh->lanes = 1;
  while (sh->lanes < kWave && sh->lanes < sh->row_vecs) sh->lanes <<= 1;
  const int64_t per_group = kThreads / sh->lanes;
  const int64_t chunks = (n + per_group - 1) / per_group;
  if (chunks * n_arrays > kMaxGrid) return false;
  sh->chunks = static_cast<int32_t>(chunks);
  sh->xcd = xcd ? 1 : 0;
  sh->groups = static_cast<int32_t>(chunks * n_arrays);
  *grid = static_cast<uint32_t>(sh->groups);
  return true;
}

int row_align(int64_t row_bytes, int pool_align, std::initializer_list<const void*> ptrs) {
  int align = 16;
  while (align > 1 && (row_bytes % align)) align >>= 1;
  align = std::min(align, pool_align);
  for (const void* p : ptrs) align = std::min(align, align_of_ptr(reinterpret_cast<uint64_t>(p)));
  return align;
}

int check_pool(const iekv_pool* p, const char* what) {
  if (!p) return set_error(IEKV_ERR_INVALID, "%s pool is null", what);
  return IEKV_OK;
}

// How two pool handles share memory: kSeparate (no byte in common), kSamePool
// (one set of arrays described twice, or one handle), or kPartial (arrays that
// overlap without being the same arrays, where block ids of one pool say
// nothing about the other's). Handles are compared by the memory they describe,
// not by identity, so two handles made over one cache count as one pool.
enum Aliasing { kSeparate = 0, kSamePool = 1, kPartial = 2 };

Aliasing pool_aliasing(const iekv_pool* a, const iekv_pool* b) {
  if (a == b) return kSamePool;
  if (a->device != b->device || a->hi <= b->lo || b->hi <= a->lo) return kSeparate;
  if (a->arrays == b->arrays && a->tile_bytes == b->tile_bytes &&
      a->num_blocks == b->num_blocks)
    return kSamePool;
  std::vector<iekv_plan::Span> spans;
  spans.reserve(a->arrays.size() + b->arrays.size());
  for (const iekv_pool* p : {a, b})
    for (uint64_t base : p->arrays)
      spans.push_back({base, base + static_cast<uint64_t>(p->num_blocks * p->tile_bytes),
                       p == a ? 0 : 1});
  return iekv_plan::spans_cross(spans) ? kPartial : kSeparate;
}

// The aliasing of a move's source and destination pools, with kPartial refused.
int check_aliasing(const iekv_pool* src, const iekv_pool* dst, bool* same_pool) {
  const Aliasing al = pool_aliasing(src, dst);
  if (al == kPartial)
    return set_error(IEKV_ERR_INVALID, "the source and destination pools overlap in memory "
                     "without being the same pool");
  *same_pool = al == kSamePool;
  return IEKV_OK;
}

int check_ids(const int32_t* ids, int32_t n_blocks, const char* what) {
  if (n_blocks < 0) return set_error(IEKV_ERR_INVALID, "n_blocks is negative (%d)", n_blocks);
  if (n_blocks > 0 && !ids) return set_error(IEKV_ERR_INVALID, "%s ids are null", what);
  return IEKV_OK;
}

int check_buffer(const void* buf, int64_t bytes, int64_t need, const char* what) {
  if (need > 0 && !buf) return set_error(IEKV_ERR_INVALID, "%s buffer is null", what);
  if (bytes < need)
    return set_error(IEKV_ERR_CAPACITY, "%s buffer holds %lld bytes, %lld needed", what,
                     static_cast<long long>(bytes), static_cast<long long>(need));
  return IEKV_OK;
}

// Bytes of n block images of pool p, or -1 on overflow.
int64_t image_bytes(const iekv_pool* p, int64_t n) {
  const int64_t block = p->tile_bytes * p->n_arrays;
  if (n > 0 && block > INT64_MAX / n) return -1;
  return block * n;
}

// Bytes from p to the end of the HIP allocation that holds it (pinned host
// memory included), or 0 when the runtime does not know p. A failed lookup is
// not an error of the caller's call, so it is cleared from HIP's last error.
int64_t bytes_to_allocation_end(const char* p) {
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<char*>(p)) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return static_cast<int64_t>(static_cast<const char*>(base) + size - p);
}

// Host transfers skip the staging buffer when the host range lies in one pinned
// allocation mapped for the device: the move kernel writes (offload) or reads
// (restore) the host buffer itself over the host link, in launches of at most
// this many bytes of images. Measured on MI355X against the staged pipelines,
// one call per request: one 2 MiB block offloads in 40 us instead of 525 us and
// restores in 52 us instead of 333 us; 64 blocks of 32 KiB move at 53 GB/s
// instead of 7 GB/s. For large images the staged pipelines' runtime copies
// reached 55-56 GB/s on some boxes but 28-39 GB/s (host to device) and 32-33
// GB/s (device to host) on others, where the direct launches held 54-57 GB/s.
constexpr int64_t kZeroCopyMaxBytes = IEKV_HOST_DIRECT_MAX_BYTES;

// Chunk size of the unpack launches that read pinned host memory themselves (the
// direct restores): 0, whole tiles per workgroup. Reads across the host link
// gain from each workgroup streaming a longer contiguous run. Measured on MI355X,
// one restore per block, bytes per second against 4 KiB chunks: 2 MiB blocks of
// 32 KiB tiles 40.5 -> 51.0 GB/s, 2.5 MiB of 16 KiB tiles 41.5 -> 50.2, 3 MiB of
// 64 KiB tiles 41.5 -> 53.7; 24 images per call 53.3 -> 56.6 on 32 KiB tiles, within
// 3% either way on the others. Writes to host memory (direct offloads) measured
// the same at either size, so they keep the staging chunk.
// Tiles smaller than the staging chunk keep it, so several of them still share
// a workgroup.
#ifndef IEKV_HOST_READ_CHUNK
#define IEKV_HOST_READ_CHUNK 0
#endif
constexpr int32_t kHostReadChunk = IEKV_HOST_READ_CHUNK;

int32_t host_read_chunk(int64_t tile_bytes) {
  const int32_t staged = g_chunk.load();
  return staged > 0 && tile_bytes < staged ? staged : kHostReadChunk;
}

// Cache policy of the pack launches that write pinned host memory themselves
// (direct offloads): ordinary loads and stores for tiles of at least
// kHostWriteTemporalTile bytes, else the setting. Measured on MI355X, offloads of
// 21-32 block images per call, ordinary against non-temporal: 1 MiB blocks of
// 16 KiB tiles 51.2 -> 54.2 GB/s, 2 MiB of 32 KiB 52.7 -> 54.5, 2.5 MiB of 16 KiB
// 52.7 -> 54.5, 3 MiB of 64 KiB 52.9 -> 54.5; 4 KiB tiles 52.9 -> 52.9 and 8 KiB
// tiles 51.6 -> 51.3; one block per call the same either way.
#ifndef IEKV_HOST_WRITE_TEMPORAL_TILE
#define IEKV_HOST_WRITE_TEMPORAL_TILE 16384
#endif
constexpr int64_t kHostWriteTemporalTile = IEKV_HOST_WRITE_TEMPORAL_TILE;

int32_t host_write_nontemporal(int64_t tile_bytes) {
  return tile_bytes >= kHostWriteTemporalTile ? 0 : -1;
}

// What HIP reports for the host allocation holding address p (iekv_plan::HostSpan):
// pinned and mapped for the device (hipPointerGetAttributes gives a pinned host
// pointer's device address), the bytes from p to the allocation's end
// (hipMemGetAddressRange), and device minus host address. Failed lookups are
// cleared from HIP's last error and report unmapped memory.
iekv_plan::HostSpan host_span(uint64_t p) {
  iekv_plan::HostSpan span;
  const void* ptr = reinterpret_cast<const void*>(p);
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return span;
  }
  if (attr.type != hipMemoryTypeHost || !attr.devicePointer || !attr.hostPointer) return span;
  span.room = bytes_to_allocation_end(static_cast<const char*>(ptr));
  span.shift = static_cast<int64_t>(reinterpret_cast<uint64_t>(attr.devicePointer) -
                                    reinterpret_cast<uint64_t>(attr.hostPointer));
  span.mapped = span.room > 0;
  return span;
}

// The device address of the host range [p, p + bytes) when it lies in one
// pinned allocation mapped for the device, else nullptr: pageable or unknown
// memory, or a range running past its allocation.
char* device_view_of_host(const void* p, int64_t bytes) {
  uint64_t view = 0;
  if (!iekv_plan::image_views(&p, 1, bytes, host_span, &view)) return nullptr;
  return reinterpret_cast<char*>(view);
}

// Device addresses of n host images of `bytes` each, when every one lies in a
// pinned allocation mapped for the device (iekv_plan::image_views: one lookup
// per allocation). False otherwise.
bool device_views_of_images(const void* const* images, int32_t n, int64_t bytes,
                            uint64_t* out) {
  return iekv_plan::image_views(images, n, bytes, host_span, out);
}

// A small set of events that lives for one pipeline call.
class Events {
 public:
  int create(int n) {
    ev_.assign(n, nullptr);
    for (auto& e : ev_) IEKV_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return IEKV_OK;
  }
  ~Events() {
    for (auto e : ev_)
      if (e) (void)hipEventDestroy(e);
  }
  hipEvent_t operator[](int i) const { return ev_[i]; }

 private:
  std::vector<hipEvent_t> ev_;
};

// -1 (keep), or a base order 0..2 with or without the kXcdGrouped flag.
bool valid_order(int32_t order) {
  if (order == -1) return true;
  return order >= 0 && order <= (kXcdGrouped | iekv_plan::kScattered);
}

// A chunk setting: -1 (keep), 0 (whole tiles) or a power of two from 64 to 1 MiB.
bool valid_chunk(int32_t chunk_bytes) {
  if (chunk_bytes == -1 || chunk_bytes == 0) return true;
  return chunk_bytes >= 64 && chunk_bytes <= (1 << 20) && !(chunk_bytes & (chunk_bytes - 1));
}

// IEKV_ERR_RANGE unless each of the n host ids lies in [0, num_blocks).
int check_host_range(const int32_t* host_ids, int32_t n, int64_t num_blocks, const char* what) {
  for (int32_t i = 0; i < n; ++i) {
    const int32_t id = host_ids[i];
    if (id < 0 || id >= num_blocks)
      return set_error(IEKV_ERR_RANGE, "%s block id %d (entry %d) out of range for a pool of "
                       "%lld blocks", what, id, i, static_cast<long long>(num_blocks));
  }
  return IEKV_OK;
}

// IEKV_ERR_IDS unless the n ids at v are distinct.
int check_distinct(const int32_t* v, int32_t n, const char* what) {
  std::vector<int32_t> sorted(v, v + n);
  std::sort(sorted.begin(), sorted.end());
  for (int32_t i = 1; i < n; ++i)
    if (sorted[i] == sorted[i - 1])
      return set_error(IEKV_ERR_IDS, "%s block ids must be distinct (id %d given twice)", what,
                       sorted[i]);
  return IEKV_OK;
}

// The checked (src, dst) pairs of a host-id direct copy, reordered by ascending
// destination id into src_out / dst_out. IEKV_ERR_IDS for a destination given
// twice, and, when both sides are the same pool, for a block that is both a
// source and a destination (its bytes would depend on the order the workgroups
// run in).
int order_pairs(const int32_t* src_ids, const int32_t* dst_ids, int32_t n, bool same_pool,
                std::vector<int32_t>* src_out, std::vector<int32_t>* dst_out) {
  std::vector<uint64_t> key(n);   // destination in the high half: sorting orders by it
  for (int32_t i = 0; i < n; ++i)
    key[i] = (static_cast<uint64_t>(static_cast<uint32_t>(dst_ids[i])) << 32) |
             static_cast<uint32_t>(src_ids[i]);
  std::sort(key.begin(), key.end());
  src_out->resize(n);
  dst_out->resize(n);
  int32_t* s = src_out->data();
  int32_t* d = dst_out->data();
  for (int32_t i = 0; i < n; ++i) {
    s[i] = static_cast<int32_t>(key[i] & 0xffffffffu);
    d[i] = static_cast<int32_t>(key[i] >> 32);
    if (i > 0 && d[i] == d[i - 1])
      return set_error(IEKV_ERR_IDS, "destination block ids must be distinct (id %d given "
                       "twice)", d[i]);
  }
  if (same_pool) {
    std::vector<int32_t> srcs(s, s + n);
    std::sort(srcs.begin(), srcs.end());
    for (int32_t i = 0, j = 0; i < n && j < n;) {   // d ascends
      if (srcs[i] == d[j])
        return set_error(IEKV_ERR_IDS, "a direct copy within one pool needs disjoint source "
                         "and destination blocks (block %d is both)", srcs[i]);
      if (srcs[i] < d[j]) ++i; else ++j;
    }
  }
  return IEKV_OK;
}

int check_host_count(int32_t n_blocks, const int32_t* a, const int32_t* b) {
  if (n_blocks < 0)
    return set_error(IEKV_ERR_INVALID, "n_blocks is negative (%d) for host ids", n_blocks);
  if (n_blocks > 0 && (!a || !b)) return set_error(IEKV_ERR_INVALID, "host ids are null");
  return IEKV_OK;
}

// A move whose (checked) ids are in host memory, in launches of at most
// IEKV_INLINE_IDS blocks that carry their ids in their kernel arguments. src_ids
// (when the source is a pool) and dst_ids (when the destination is) hold
// n_blocks ids; staging images follow the list order.
template <bool SP, bool DP>
int launch_host_ids(const iekv_pool* sp, const iekv_pool* dp, const char* src_stage,
                    char* dst_stage, const int32_t* src_ids, const int32_t* dst_ids,
                    int32_t n_blocks, int64_t tile_bytes, int32_t n_arrays, int align,
                    hipStream_t stream, int32_t chunk = -1, int32_t nt = -1,
                    bool host = false) {
  const int64_t image = tile_bytes * n_arrays;
  // One launch's m ids in an id block of W words: sources first, then destinations.
  auto launch = [&](auto words, int32_t first, int32_t m) {
    constexpr int W = decltype(words)::value;
    InlineIds<W> ids{};
    int32_t dst_off = 0;
    if (SP) {
      std::copy(src_ids + first, src_ids + first + m, ids.v);
      dst_off = m;
    }
    if (DP) std::copy(dst_ids + first, dst_ids + first + m, ids.v + dst_off);
    return launch_move_inline<SP, DP, W>(
        sp, dp, SP ? nullptr : src_stage + first * image, DP ? nullptr : dst_stage + first * image,
        ids, dst_off, m, tile_bytes, n_arrays, align, stream, chunk, nt, host);
  };
  constexpr int32_t kWordsPerId = (SP ? 1 : 0) + (DP ? 1 : 0);
  for (int32_t first = 0; first < n_blocks; first += IEKV_INLINE_IDS) {
    const int32_t m = std::min<int32_t>(IEKV_INLINE_IDS, n_blocks - first);
    const int rc = m * kWordsPerId <= kSmallIdWords
                       ? launch(std::integral_constant<int, kSmallIdWords>{}, first, m)
                       : launch(std::integral_constant<int, kIdWords>{}, first, m);
    if (rc) return rc;
  }
  return IEKV_OK;
}


// The block ids of a host pipeline call: in device memory (the kernels read
// them) or in host memory (checked before the call, then carried in the
// launches' kernel arguments, IEKV_INLINE_IDS per launch).
struct IdList {
  const int32_t* ids;
  bool on_host;
  IdList from(int64_t first) const { return {ids + first, on_host}; }
};

// A pack (SP: pool -> staging) or unpack (DP: staging -> pool) of n_blocks
// blocks of `pool` whose ids are an IdList.
template <bool SP, bool DP>
int launch_list(const iekv_pool* pool, const char* src_stage, char* dst_stage, IdList list,
                int32_t n_blocks, int align, hipStream_t stream, int32_t chunk = -1,
                int32_t nt = -1, bool host = false) {
  static_assert(SP != DP, "a pack or an unpack");
  const iekv_pool* sp = SP ? pool : nullptr;
  const iekv_pool* dp = DP ? pool : nullptr;
  const int32_t* s = SP ? list.ids : nullptr;
  const int32_t* d = DP ? list.ids : nullptr;
  if (list.on_host)
    return launch_host_ids<SP, DP>(sp, dp, src_stage, dst_stage, s, d, n_blocks,
                                   pool->tile_bytes, pool->n_arrays, align, stream, chunk, nt,
                                   host);
  return launch_move<SP, DP>(sp, dp, src_stage, dst_stage, s, d, n_blocks, pool->tile_bytes,
                             pool->n_arrays, align, stream, chunk, nt, host);
}

// Restore pipeline shared by the iekv_restore* calls: chunk k of the blocks is
// copied from host memory into a staging slot on `copy` (by
// `load(slot, first, count)`) while `compute` unpacks chunk k-1 onto dst_ids.
// Two slots when the staging buffer holds two blocks or more, else one.
template <typename Load>
int restore_pipeline(const iekv_pool* dst, IdList dst_ids, int32_t n_blocks,
                     void* staging, int64_t staging_bytes, hipStream_t compute,
                     hipStream_t copy, Load load) {
  int rc;
  const int64_t block_bytes = image_bytes(dst, 1);
  if ((rc = check_buffer(staging, staging_bytes, n_blocks ? block_bytes : 0, "staging")))
    return rc;
  if (n_blocks == 0) return IEKV_OK;
  DeviceGuard guard(dst->device);
  if (!guard.ok()) return guard.fail();

  int n_slots;
  int64_t slot_blocks;
  if (!iekv_plan::plan_slots(staging_bytes, block_bytes, n_blocks, &n_slots, &slot_blocks))
    return set_error(IEKV_ERR_CAPACITY, "staging buffer holds no block image");
  const int align =
      std::min(dst->align, align_of_ptr(reinterpret_cast<uint64_t>(staging)));
  Events loaded, unpacked, fence;
  if ((rc = loaded.create(n_slots)) || (rc = unpacked.create(n_slots)) || (rc = fence.create(1)))
    return rc;

  // Entry fence: the copy stream must not overwrite staging while earlier
  // compute-stream work still reads it.
  IEKV_HIP(hipEventRecord(fence[0], compute));
  IEKV_HIP(hipStreamWaitEvent(copy, fence[0], 0));

  char* stage = static_cast<char*>(staging);
  int last = 0;
  for (int64_t first = 0, k = 0; first < n_blocks; first += slot_blocks, ++k) {
    const int32_t cnt = static_cast<int32_t>(std::min<int64_t>(slot_blocks, n_blocks - first));
    const int s = static_cast<int>(k % n_slots);
    char* slot = stage + s * slot_blocks * block_bytes;
    if (k >= n_slots) IEKV_HIP(hipStreamWaitEvent(copy, unpacked[s], 0));
    if ((rc = load(slot, first, cnt))) return rc;
    IEKV_HIP(hipEventRecord(loaded[s], copy));
    IEKV_HIP(hipStreamWaitEvent(compute, loaded[s], 0));
    if ((rc = launch_list<false, true>(dst, slot, nullptr, dst_ids.from(first), cnt, align,
                                       compute)))
      return rc;
    IEKV_HIP(hipEventRecord(unpacked[s], compute));
    last = s;
  }
  // Later copy-stream work that writes staging is ordered after the last unpack.
  IEKV_HIP(hipStreamWaitEvent(copy, unpacked[last], 0));
  return IEKV_OK;
}

// Events of one offload pipeline call: per staging slot, "packed" (recorded on
// the compute stream after the slot's pack) and "copied" (on the copy stream
// after its device-to-host copy), plus the entry fence. `last` is the slot
// whose "copied" event the previous call through these events recorded last
// (-1 before the first): a call that shares the staging buffer with earlier
// calls makes its compute stream wait on it, so its packs never overwrite a
// slot an earlier call's device-to-host copy still reads, whatever streams the
// two calls run on.
struct OffloadEvents {
  hipEvent_t packed[2];
  hipEvent_t copied[2];
  hipEvent_t fence;
  int last = -1;
};

// Arguments of an offload, checked before anything touches the GPU; *need is
// the host image size.
int check_offload(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                  const void* host_dst, int64_t host_bytes, int64_t* need) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_ids(src_ids, n_blocks, "source")))
    return rc;
  *need = image_bytes(src, n_blocks);
  if (*need < 0) return set_error(IEKV_ERR_INVALID, "host image size overflows");
  return check_buffer(host_dst, host_bytes, *need, "host");
}

// The staged offload of n_blocks >= 1 checked blocks with src's device
// current: chunk k is packed into a staging slot on `compute` while `copy`
// moves chunk k-1 to the host with store(slot, first, count) (two slots when
// the staging holds two blocks or more, else one). `preset` gives the events
// to use, and is ordered after the previous call that used them (its `last`
// is updated); without it the call creates its own.
template <typename Store>
int offload_pipeline(const iekv_pool* src, IdList src_ids, int32_t n_blocks, char* staging,
                     int64_t staging_bytes, hipStream_t compute, hipStream_t copy,
                     OffloadEvents* preset, Store store) {
  int rc;
  const int64_t block_bytes = image_bytes(src, 1);
  if ((rc = check_buffer(staging, staging_bytes, block_bytes, "staging"))) return rc;
  int n_slots;
  int64_t slot_blocks;
  if (!iekv_plan::plan_slots(staging_bytes, block_bytes, n_blocks, &n_slots, &slot_blocks))
    return set_error(IEKV_ERR_CAPACITY, "staging buffer holds no block image");
  const int align = std::min(src->align, align_of_ptr(reinterpret_cast<uint64_t>(staging)));
  Events own;
  OffloadEvents ev{};
  if (preset) {
    ev = *preset;
  } else {
    if ((rc = own.create(2 * n_slots + 1))) return rc;
    for (int s = 0; s < n_slots; ++s) {
      ev.packed[s] = own[2 * s];
      ev.copied[s] = own[2 * s + 1];
    }
    ev.fence = own[2 * n_slots];
  }

  // A shared staging buffer: the previous call's last device-to-host copy
  // comes after all of its packs and copies, so waiting on it frees every slot.
  if (preset && preset->last >= 0)
    IEKV_HIP(hipStreamWaitEvent(compute, ev.copied[preset->last], 0));
  // Entry fence: the copy stream must not read staging before the compute
  // stream's earlier work on it has finished.
  IEKV_HIP(hipEventRecord(ev.fence, compute));
  IEKV_HIP(hipStreamWaitEvent(copy, ev.fence, 0));

  int last = 0;
  for (int64_t first = 0, k = 0; first < n_blocks; first += slot_blocks, ++k) {
    const int32_t cnt = static_cast<int32_t>(std::min<int64_t>(slot_blocks, n_blocks - first));
    const int s = static_cast<int>(k % n_slots);
    char* slot = staging + s * slot_blocks * block_bytes;
    if (k >= n_slots) IEKV_HIP(hipStreamWaitEvent(compute, ev.copied[s], 0));
    if ((rc = launch_list<true, false>(src, nullptr, slot, src_ids.from(first), cnt, align,
                                       compute)))
      return rc;
    IEKV_HIP(hipEventRecord(ev.packed[s], compute));
    IEKV_HIP(hipStreamWaitEvent(copy, ev.packed[s], 0));
    if ((rc = store(slot, first, cnt))) return rc;
    IEKV_HIP(hipEventRecord(ev.copied[s], copy));
    last = s;
    if (preset) preset->last = s;
  }
  // Later compute-stream work (reuse of staging, reads of the host images after
  // a sync of `compute`) is ordered after the last device-to-host copy.
  IEKV_HIP(hipStreamWaitEvent(compute, ev.copied[last], 0));
  return IEKV_OK;
}

// The offload of n_blocks >= 1 checked blocks into one host image, with src's
// device current. An image in one pinned, device-mapped allocation is written by
// the pack kernel directly, whatever its size, in launches of at most
// kZeroCopyMaxBytes of images; otherwise (pageable memory) the staged pipeline
// copies each chunk with one hipMemcpyAsync. Measured on MI355X, 4 GiB of 2 MiB
// block images into pinned memory: the direct launches moved 54.4 GB/s in every
// round on a box where the staged pipeline's device-to-host copies moved
// 32-33 GB/s (on another box they had reached 56.6).
int run_offload(const iekv_pool* src, IdList src_ids, int32_t n_blocks, void* host_dst,
                int64_t need, char* staging, int64_t staging_bytes, hipStream_t compute,
                hipStream_t copy, OffloadEvents* preset) {
  const int64_t block_bytes = image_bytes(src, 1);
  if (char* mapped = device_view_of_host(host_dst, need)) {
    const int32_t per =
        iekv_plan::images_per_launch(n_blocks, block_bytes, kZeroCopyMaxBytes, INT32_MAX);
    const int32_t nt = host_write_nontemporal(src->tile_bytes);
    for (int32_t first = 0; first < n_blocks; first += per) {
      const int32_t cnt = std::min(per, n_blocks - first);
      char* piece = mapped + first * block_bytes;
      const int zc_align = std::min(src->align, align_of_ptr(reinterpret_cast<uint64_t>(piece)));
      const int rc = launch_list<true, false>(src, nullptr, piece, src_ids.from(first), cnt,
                                              zc_align, compute, -1, nt);
      if (rc) return rc;
    }
    return IEKV_OK;
  }
  char* host = static_cast<char*>(host_dst);
  return offload_pipeline(src, src_ids, n_blocks, staging, staging_bytes, compute, copy, preset,
                          [&](char* slot, int64_t first, int32_t cnt) -> int {
                            IEKV_HIP(hipMemcpyAsync(host + first * block_bytes, slot,
                                                    cnt * block_bytes, hipMemcpyDeviceToHost,
                                                    copy));
                            return IEKV_OK;
                          });
}

// The staging of iekv_offload_static on one device: the device address of
// `scratch` there and the pipeline's events, set up by the first call on
// that device and kept until the process ends. g_static_mu is held for the
// whole of each call's enqueueing, so calls from several host threads are
// enqueued one after another, each ordered on the device after the previous
// one's copies (OffloadEvents::last).
struct StaticStaging {
  bool ready = false;
  char* ptr = nullptr;
  OffloadEvents events{};
};
constexpr int kMaxStaticDevices = 64;
std::mutex g_static_mu;
StaticStaging g_static[kMaxStaticDevices];

// The static staging of `device`, which must be the current device; the caller
// holds g_static_mu.
int static_staging(int device, StaticStaging** out) {
  if (device < 0 || device >= kMaxStaticDevices)
    return set_error(IEKV_ERR_INVALID, "device %d is outside 0..%d", device,
                     kMaxStaticDevices - 1);
  StaticStaging& st = g_static[device];
  if (!st.ready) {
    // `scratch` names the host-side stand-in of the device array; the address
    // kernels may use is the one HIP reports for the current device.
    void* addr = nullptr;
    IEKV_HIP(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
    if (!addr) return set_error(IEKV_ERR_HIP, "hipGetSymbolAddress gave a null address");
    hipEvent_t ev[5] = {};
    for (int i = 0; i < 5; ++i) {
      const hipError_t e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
        return set_error(IEKV_ERR_HIP, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
      }
    }
    st.events = OffloadEvents{{ev[0], ev[1]}, {ev[2], ev[3]}, ev[4]};
    st.ptr = static_cast<char*>(addr);
    st.ready = true;
  }
  *out = &st;
  return IEKV_OK;
}

// `copy` ordered after the work enqueued so far on `compute` (the end state of
// every restore: the staging buffer and the host images may then be reused on
// either stream).
int order_copy_after(hipStream_t compute, hipStream_t copy) {
  if (copy == compute) return IEKV_OK;
  int rc;
  Events done;
  if ((rc = done.create(1))) return rc;
  IEKV_HIP(hipEventRecord(done[0], compute));
  IEKV_HIP(hipStreamWaitEvent(copy, done[0], 0));
  return IEKV_OK;
}

// iekv_restore / iekv_restore_ids after their id checks: one contiguous host
// image of n_blocks block images onto dst_ids. An image in one pinned,
// device-mapped allocation is read by the unpack kernel itself, whatever its
// size, in launches of at most kZeroCopyMaxBytes of images; pageable or
// unknown memory goes through the staged pipeline.
int restore_image(const iekv_pool* dst, IdList dst_ids, int32_t n_blocks, const void* host_src,
                  int64_t host_bytes, void* staging, int64_t staging_bytes, hipStream_t compute,
                  hipStream_t copy) {
  int rc;
  const int64_t need = image_bytes(dst, n_blocks);
  if (need < 0) return set_error(IEKV_ERR_INVALID, "host image size overflows");
  if ((rc = check_buffer(host_src, host_bytes, need, "host"))) return rc;
  const int64_t block_bytes = image_bytes(dst, 1);
  if (n_blocks > 0) {
    DeviceGuard guard(dst->device);
    if (!guard.ok()) return guard.fail();
    if (const char* mapped = device_view_of_host(host_src, need)) {
      const int32_t per =
          iekv_plan::images_per_launch(n_blocks, block_bytes, kZeroCopyMaxBytes, INT32_MAX);
      const int32_t chunk = host_read_chunk(dst->tile_bytes);
      for (int32_t first = 0; first < n_blocks; first += per) {
        const int32_t cnt = std::min(per, n_blocks - first);
        const char* piece = mapped + first * block_bytes;
        const int zc_align = std::min(dst->align, align_of_ptr(reinterpret_cast<uint64_t>(piece)));
        if ((rc = launch_list<false, true>(dst, piece, nullptr, dst_ids.from(first), cnt,
                                           zc_align, compute, chunk, -1, true)))
          return rc;
      }
      // As after the staged pipeline, `copy` is ordered after the last unpack.
      return order_copy_after(compute, copy);
    }
  }
  const char* host = static_cast<const char*>(host_src);
  return restore_pipeline(
      dst, dst_ids, n_blocks, staging, staging_bytes, compute, copy,
      [&](char* slot, int64_t first, int32_t cnt) -> int {
        IEKV_HIP(hipMemcpyAsync(slot, host + first * block_bytes, cnt * block_bytes,
                                hipMemcpyHostToDevice, copy));
        return IEKV_OK;
      });
}

// iekv_offload_blocks / iekv_offload_blocks_ids after their id checks: block
// src_ids[i] packed into the host image at host_blocks[i]. When every image lies
// in pinned, device-mapped memory, pack launches write them directly, up to
// IEKV_INLINE_IMAGES images and kZeroCopyMaxBytes per launch (their addresses
// in the kernel arguments); otherwise the staged pipeline copies each run of
// images adjacent within one allocation with one hipMemcpyAsync.
int offload_images(const iekv_pool* src, IdList src_ids, int32_t n_blocks,
                   void* const* host_blocks, void* staging, int64_t staging_bytes,
                   hipStream_t compute, hipStream_t copy) {
  int rc;
  if (n_blocks > 0 && !host_blocks)
    return set_error(IEKV_ERR_INVALID, "host block address list is null");
  for (int32_t i = 0; i < n_blocks; ++i)
    if (!host_blocks[i]) return set_error(IEKV_ERR_INVALID, "host block %d address is null", i);
  const int64_t block_bytes = image_bytes(src, 1);
  if (n_blocks == 0) return IEKV_OK;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  const int32_t per = iekv_plan::images_per_launch(n_blocks, block_bytes, kZeroCopyMaxBytes,
                                                   IEKV_INLINE_IMAGES);
  // Every image's device address first: the call goes direct only if all of them
  // have one, so it never mixes the two paths.
  std::vector<uint64_t> views(n_blocks);
  bool direct = true;
  for (int32_t first = 0; direct && first < n_blocks; first += per)
    direct = device_views_of_images(host_blocks + first, std::min(per, n_blocks - first),
                                    block_bytes, views.data() + first);
  if (direct) {
    const int32_t nt = host_write_nontemporal(src->tile_bytes);
    for (int32_t first = 0; first < n_blocks; first += per) {
      const int32_t cnt = std::min(per, n_blocks - first);
      InlineImages images{};
      std::copy(views.begin() + first, views.begin() + first + cnt, images.addr);
      const int32_t* device_ids = src_ids.on_host ? nullptr : src_ids.ids + first;
      if (src_ids.on_host) std::copy(src_ids.ids + first, src_ids.ids + first + cnt, images.ids);
      if ((rc = launch_images<true, false>(src, images, device_ids, cnt, compute, -1, nt)))
        return rc;
    }
    return IEKV_OK;
  }
  return offload_pipeline(
      src, src_ids, n_blocks, static_cast<char*>(staging), staging_bytes, compute, copy, nullptr,
      [&](char* slot, int64_t first, int32_t cnt) -> int {
        hipError_t err = hipSuccess;
        iekv_plan::image_runs(
            host_blocks + first, cnt, block_bytes,
            [](uint64_t address) {
              return bytes_to_allocation_end(reinterpret_cast<const char*>(address));
            },
            [&](int32_t i, int32_t len) {
              if (err == hipSuccess)
                err = hipMemcpyAsync(host_blocks[first + i], slot + i * block_bytes,
                                     len * block_bytes, hipMemcpyDeviceToHost, copy);
            });
        IEKV_HIP(err);
        return IEKV_OK;
      });
}

// iekv_restore_blocks / iekv_restore_blocks_ids after their id checks: block
// image i at host_blocks[i] onto dst_ids[i]. When every image lies in a pinned,
// device-mapped allocation, the unpack kernel reads them itself, in launches
// of at most IEKV_INLINE_IMAGES images and kZeroCopyMaxBytes (their addresses
// in the kernel arguments); otherwise the staged pipeline copies them.
int restore_images(const iekv_pool* dst, IdList dst_ids, int32_t n_blocks,
                   const void* const* host_blocks, void* staging, int64_t staging_bytes,
                   hipStream_t compute, hipStream_t copy) {
  int rc;
  if (n_blocks > 0 && !host_blocks)
    return set_error(IEKV_ERR_INVALID, "host block address list is null");
  for (int32_t i = 0; i < n_blocks; ++i)
    if (!host_blocks[i]) return set_error(IEKV_ERR_INVALID, "host block %d address is null", i);
  const int64_t block_bytes = image_bytes(dst, 1);
  if (n_blocks > 0) {
    DeviceGuard guard(dst->device);
    if (!guard.ok()) return guard.fail();
    const int32_t per = iekv_plan::images_per_launch(n_blocks, block_bytes, kZeroCopyMaxBytes,
                                                     IEKV_INLINE_IMAGES);
    // Every image's device address first: the call goes direct only if all of them
    // have one, so it never mixes the two paths.
    std::vector<uint64_t> views(n_blocks);
    bool direct = true;
    for (int32_t first = 0; direct && first < n_blocks; first += per)
      direct = device_views_of_images(host_blocks + first, std::min(per, n_blocks - first),
                                      block_bytes, views.data() + first);
    if (direct) {
      const int32_t chunk = host_read_chunk(dst->tile_bytes);
      for (int32_t first = 0; first < n_blocks; first += per) {
        const int32_t cnt = std::min(per, n_blocks - first);
        InlineImages images{};
        std::copy(views.begin() + first, views.begin() + first + cnt, images.addr);
        const int32_t* device_ids = dst_ids.on_host ? nullptr : dst_ids.ids + first;
        if (dst_ids.on_host) std::copy(dst_ids.ids + first, dst_ids.ids + first + cnt, images.ids);
        if ((rc = launch_images<false, true>(dst, images, device_ids, cnt, compute, chunk, -1,
                                             true)))
          return rc;
      }
      // As after the staged pipeline, `copy` is ordered after the last unpack.
      return order_copy_after(compute, copy);
    }
  }
  return restore_pipeline(
      dst, dst_ids, n_blocks, staging, staging_bytes, compute, copy,
      [&](char* slot, int64_t first, int32_t cnt) -> int {
        // One copy per run of images that are adjacent in host memory within
        // one allocation (iekv_plan::image_runs).
        hipError_t err = hipSuccess;
        iekv_plan::image_runs(
            host_blocks + first, cnt, block_bytes,
            [](uint64_t address) {
              return bytes_to_allocation_end(reinterpret_cast<const char*>(address));
            },
            [&](int32_t i, int32_t len) {
              if (err == hipSuccess)
                err = hipMemcpyAsync(slot + i * block_bytes, host_blocks[first + i],
                                     len * block_bytes, hipMemcpyHostToDevice, copy);
            });
        IEKV_HIP(err);
        return IEKV_OK;
      });
}

// ---------------------------------------------------------------------------
// Request queue (iekv_queue_*): a resident kernel serving direct handoffs
// ---------------------------------------------------------------------------
// The host writes descriptor r (a header and the request's ids) into slot
// r % kQueueSlots of a ring in pinned, coherent host memory and publishes it by
// raising `tail` to r + 1. Workgroup 0 of the kernel (the leader) polls `tail`,
// reads each new descriptor, writes one record per claim of it (its block's id
// pair and units, iekv_plan::queue_claims) into the device's claim ring, sets
// the slot's `remaining` count, and raises `published_claims`. The waves of the
// other workgroups (movers) take claim numbers from a set of cursors, wait until
// their claim is published, read its record, move its units, and count it down
// in the slot's `remaining` word; the mover that finishes a descriptor's last
// claim writes r + 1 into the slot's `complete` word in host memory. The host
// reuses a slot only after its descriptor is complete, so no slot is rewritten
// while its descriptor is served, and the claim ring holds twice the claims of
// every descriptor in flight, so no record is rewritten while its claim waits.
// Every wait ends: the leader's poll and a mover's wait for its claim both end
// on the stop flag, after idle_ticks without a new descriptor, or life_ticks
// after the workgroup started. The host keeps its submissions inside half of
// each limit (queue_publish), so no descriptor is published to a kernel that
// may be ending.
constexpr int kQueueSlots = IEKV_QUEUE_SLOTS;
constexpr int kQueueBlocks = IEKV_QUEUE_MAX_BLOCKS;
constexpr int64_t kQueueClaimRing = iekv_plan::queue_claim_ring(kQueueSlots);

// One descriptor as the host writes it (k, per_block and n_claims from
// iekv_plan::queue_claims).
struct QueueHeader {
  uint64_t claim_base;   // the descriptor's first claim in its session
  int32_t n_blocks;
  int32_t n_claims;
  int32_t k;             // units per claim
  int32_t per_block;     // claims per block
  int64_t reserved;
};

// A claim as the leader publishes it: the block's id pair, its units, and the
// descriptor it belongs to (its number in the session).
struct QueueClaim {
  int32_t src_id, dst_id;
  uint32_t units;        // first unit | unit count << 16
  uint32_t desc;
};
constexpr int32_t kQueueMaxUnits = 32768;   // units per block, so both fit 16 bits

// Pinned host memory, mapped for the device. The host writes tail, stop,
// stop_claims, the headers and the ids; the device writes `complete`.
struct QueueRing {
  alignas(64) uint64_t tail;
  alignas(64) uint64_t stop;
  uint64_t stop_claims;
  alignas(64) uint64_t complete[kQueueSlots];
  alignas(64) QueueHeader header[kQueueSlots];
  alignas(64) int32_t ids[kQueueSlots][2 * kQueueBlocks];  // sources, destinations at +kQueueBlocks
};

// Claims of a slot's descriptor not yet finished, one cache line per slot: the
// movers of neighbouring descriptors count down concurrently.
struct alignas(128) QueueCount {
  uint64_t left;
};

// Movers take claims from kQueueCursors cursors, cursor p handing out claims p,
// p + kQueueCursors, ...: each cursor is updated by a 1/kQueueCursors share of
// the movers, and any running mover keeps its cursor's claims moving.
constexpr int kQueueCursors = 32;

// Device memory. Everything before `claims` is cleared when a session starts.
struct QueueState {
  alignas(128) uint64_t published_claims;
  uint64_t stop;
  uint64_t stop_claims;
  QueueCount cursor[kQueueCursors];
  QueueCount remaining[kQueueSlots];
  alignas(128) QueueClaim claims[kQueueClaimRing];
};

struct QueueArgs {
  PoolView src, dst;
  QueueState* state;
  QueueRing* ring;         // the device's address of the host ring
  int32_t tile_vecs;
  int32_t n_arrays;
  int32_t group;           // tiles per unit (small tiles are moved in groups)
  int32_t units_per_block;
  uint64_t idle_ticks;     // wall-clock ticks
  uint64_t life_ticks;
};

// A word of the host ring, read over the host link as the host last wrote it.
template <typename T>
__device__ __forceinline__ T host_word(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A word of the device ring, after the acquire that made it visible. An atomic
// load is always a vector load: a plain one of a uniform address may be read
// through the scalar cache, which an acquire does not refresh, and a slot's
// words change between descriptors.
template <typename T>
__device__ __forceinline__ T ring_word(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <typename T>
__device__ __forceinline__ T agent_word(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A pause of about 0.25 us per unit (s_sleep 8 is 512 clocks).
__device__ __forceinline__ void queue_nap(int units) {
  for (int i = 0; i < units; ++i) __builtin_amdgcn_s_sleep(8);
}

__device__ __forceinline__ bool queue_expired(const QueueArgs& q, uint64_t start,
                                              uint64_t last) {
  const uint64_t now = wall_clock64();
  return now - last > q.idle_ticks || now - start > q.life_ticks;
}

// Device-coherent stores: agent-scope atomic stores, which the compiler issues
// with the device-coherence bit (sc1), so the data is written through the XCD's
// L2 to where every XCD reads it. Once such stores are complete (the
// vector-memory counter at zero, queue_stores_done) other workgroups may rely on
// them, without the agent-scope release fence that would write back the whole L2
// of the XCD.
template <typename T>
__device__ __forceinline__ void coherent_store(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every store this lane made is complete. The empty asm statements keep the
// compiler from moving memory accesses across the wait.
__device__ __forceinline__ void queue_stores_done() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  __asm__ __volatile__("" ::: "memory");
}

// Inclusive sum of v over the workgroup's threads (`scratch`: kThreads words of LDS).
__device__ int64_t workgroup_scan(int64_t v, int64_t* scratch) {
  const int t = threadIdx.x;
  scratch[t] = v;
  __syncthreads();
  for (int d = 1; d < kThreads; d <<= 1) {
    const int64_t add = t >= d ? scratch[t - d] : 0;
    __syncthreads();
    scratch[t] += add;
    __syncthreads();
  }
  return scratch[t];
}

// The last of the first `count` entries of ascending `first` that is at most w.
__device__ __forceinline__ int owner_of(const int64_t* first, int count, int64_t w) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (first[mid] <= w) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

static_assert(kQueueSlots <= kThreads, "the leader reads every new header at once");
constexpr int kLeaderBatch = 8;   // host-ring words in flight per lane

// Workgroup 0: publish the host's descriptors to the movers. Every descriptor
// published since the last round is fetched at once: one header per thread, then
// the ids over one index space spanning them all, so a round costs two trips over
// the host link however many descriptors it brings. Each block's id pair goes
// straight into the records of its claims, written with device-coherent stores;
// published_claims is raised once they are complete.
__device__ void queue_leader(const QueueArgs& q, uint64_t start) {
  __shared__ uint64_t s_word[2];
  __shared__ QueueHeader s_head[kQueueSlots];
  __shared__ int64_t s_scan[kThreads];
  __shared__ int64_t s_first[kThreads];   // first block of each new descriptor
  __shared__ int64_t s_claim[kThreads];   // first claim of each new descriptor
  const int t = threadIdx.x;
  QueueState* st = q.state;
  const QueueRing* ring = q.ring;
  uint64_t published = 0, last = start;
  int nap = 1;
  for (;;) {
    if (t == 0) {
      // stop before tail: a stop the host raised after its last tail is seen
      // together with that tail.
      s_word[0] = __hip_atomic_load(&ring->stop, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
      s_word[1] = __hip_atomic_load(&ring->tail, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    const uint64_t stop = s_word[0], tail = s_word[1];
    __syncthreads();
    if (tail > published) {
      // The host has at most kQueueSlots descriptors unfinished, so at most that
      // many are new.
      const int fresh = static_cast<int>(min<uint64_t>(tail - published, kQueueSlots));
      int32_t n_blocks = 0, n_claims = 0;
      if (t < fresh) {
        // Clamped to what the rings hold, so no index derived from a header can
        // leave them.
        const int slot = static_cast<int>((published + t) % kQueueSlots);
        const QueueHeader* h = &ring->header[slot];
        QueueHeader v{};
        v.claim_base = host_word(&h->claim_base);
        n_blocks = min(max(host_word(&h->n_blocks), 0), kQueueBlocks);
        v.per_block = min(max(host_word(&h->per_block), 1), q.units_per_block);
        v.k = min(max(host_word(&h->k), 1), q.units_per_block);
        n_claims = min(max(host_word(&h->n_claims), 0),
                       min(n_blocks * v.per_block, static_cast<int32_t>(iekv_plan::kQueueMaxClaims)));
        v.n_blocks = n_blocks;
        v.n_claims = n_claims;
        s_head[t] = v;
        coherent_store(&st->remaining[slot].left, static_cast<uint64_t>(n_claims));
      }
      // The new descriptors' blocks over one index space (s_first: each one's first
      // block), and their claims, which follow each other from the first one's base
      // (s_claim: each one's first claim).
      const int64_t blocks_end = workgroup_scan(n_blocks, s_scan);
      s_first[t] = blocks_end - n_blocks;
      __syncthreads();
      const int64_t total_blocks = s_scan[kThreads - 1];
      const int64_t claims_end = workgroup_scan(n_claims, s_scan);
      s_claim[t] = claims_end - n_claims;
      __syncthreads();
      const int64_t total_claims = s_scan[kThreads - 1];
      const uint64_t base = s_head[0].claim_base;
      // Block w's id pair from the host ring, kLeaderBatch blocks in flight per lane,
      // then the records of its claims: claim c of a descriptor is block
      // c / per_block, units (c % per_block) * k onward.
      for (int64_t w0 = 0; w0 < total_blocks; w0 += kThreads * kLeaderBatch) {
        int32_t src_id[kLeaderBatch], dst_id[kLeaderBatch];
#pragma unroll
        for (int b = 0; b < kLeaderBatch; ++b) {
          const int64_t w = w0 + b * kThreads + t;
          if (w < total_blocks) {
            const int i = owner_of(s_first, fresh, w);
            const int j = static_cast<int>(w - s_first[i]);
            const int32_t* from = ring->ids[(published + i) % kQueueSlots];
            src_id[b] = host_word(&from[j]);
            dst_id[b] = host_word(&from[kQueueBlocks + j]);
          }
        }
#pragma unroll
        for (int b = 0; b < kLeaderBatch; ++b) {
          const int64_t w = w0 + b * kThreads + t;
          if (w < total_blocks) {
            const int i = owner_of(s_first, fresh, w);
            const QueueHeader& h = s_head[i];
            const int32_t block = static_cast<int32_t>(w - s_first[i]);
            const uint64_t ids = static_cast<uint64_t>(static_cast<uint32_t>(src_id[b])) |
                                 (static_cast<uint64_t>(static_cast<uint32_t>(dst_id[b])) << 32);
            const uint64_t desc = (published + i) << 32;
            for (int32_t p = 0; p < h.per_block; ++p) {
              const int64_t c = static_cast<int64_t>(block) * h.per_block + p;
              if (c >= h.n_claims) break;
              const int32_t first = min(p * h.k, q.units_per_block);
              const int32_t count = min(h.k, q.units_per_block - first);
              uint64_t* rec = reinterpret_cast<uint64_t*>(
                  &st->claims[(base + s_claim[i] + c) % kQueueClaimRing]);
              coherent_store(rec, ids);
              coherent_store(rec + 1, desc | static_cast<uint32_t>(first) |
                                          (static_cast<uint64_t>(count) << 16));
            }
          }
        }
      }
      queue_stores_done();
      __syncthreads();
      if (t == 0)
        __hip_atomic_store(&st->published_claims, base + total_claims, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      published += fresh;
      last = wall_clock64();
      nap = 1;
      continue;
    }
    if (stop) {
      if (t == 0) {
        __hip_atomic_store(&st->stop_claims, host_word(&ring->stop_claims), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&st->stop, uint64_t{1}, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
    if (queue_expired(q, start, last)) return;
    queue_nap(nap);
    nap = nap < 16 ? 2 * nap : 16;
  }
}

// Stores a mover makes to destination tiles are device-coherent (see
// coherent_store). Whole tiles of 16-byte vectors are written through a buffer
// resource spanning the tile, with 16-byte stores carrying the coherence bit
// (kQueueStorePolicy); other tiles with agent-scope atomic stores of 8 bytes or
// less, a 16-byte vector as two.
constexpr bool kQueueTileBufferStores = true;
constexpr int kQueueStorePolicy = 16;        // sc1: device-coherent
constexpr int kBufferWordFormat = 0x00020000;   // buffer resource word 3: 32-bit data format

template <typename V>
__device__ __forceinline__ void queue_store(gptr<V> p, V v) {
  if constexpr (sizeof(V) == 16) {
    uint64_t w[2];
    __builtin_memcpy(w, &v, 16);
    gptr<uint64_t> d = (gptr<uint64_t>)p;
    __hip_atomic_store(d, w[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(d + 1, w[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (sizeof(V) == 8) {
    uint64_t w;
    __builtin_memcpy(&w, &v, 8);
    __hip_atomic_store((gptr<uint64_t>)p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// An address every lane of the wave holds, marked uniform for the compiler (it
// cannot see that a value read from LDS at one address is the same in every
// lane), so a buffer resource built on it lives in scalar registers.
__device__ __forceinline__ char* wave_uniform(char* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<char*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Move unit a of a block (tile a, or tiles a * group .. of a group) from block
// src_id of the source pool to block dst_id of the destination, with the lanes of
// one wave: lane l moves vectors l, l + kWave, ..., U loads in flight before their
// stores. An id outside its pool moves nothing.
template <typename V, int U, bool NT>
__device__ __forceinline__ void queue_move_unit(const QueueArgs& q, int32_t src_id,
                                                int32_t dst_id, int a) {
  if (src_id < 0 || src_id >= q.src.num_blocks || dst_id < 0 || dst_id >= q.dst.num_blocks)
    return;
  const int64_t tile_bytes = static_cast<int64_t>(q.tile_vecs) * sizeof(V);
  const int l = threadIdx.x % kWave;
  if (q.group == 1) {
    const gptr<const V> s = as_global<V>(wave_uniform(array_base(q.src, a) + src_id * tile_bytes));
    char* d = wave_uniform(array_base(q.dst, a) + dst_id * tile_bytes);
    auto store = [&](int v, V r) {
      if constexpr (sizeof(V) == 16 && kQueueTileBufferStores) {
        // tile_bytes <= kMaxTileBytes: the tile's offsets fit the resource.
        const __amdgpu_buffer_rsrc_t tile = __builtin_amdgcn_make_buffer_rsrc(
            d, 0, static_cast<int32_t>(tile_bytes), kBufferWordFormat);
        __builtin_amdgcn_raw_buffer_store_b128(r, tile, v * 16, 0, kQueueStorePolicy);
      } else {
        queue_store(as_global<V>(d) + v, r);
      }
    };
    const int full = q.tile_vecs - (U - 1) * kWave;   // v < full: all U vectors in range
    int v = l;
    for (; v < full; v += U * kWave) {
      V r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) r[u] = load_vec<V, NT>(s + v + u * kWave);
#pragma unroll
      for (int u = 0; u < U; ++u) store(v + u * kWave, r[u]);
    }
    if (v < q.tile_vecs) {
      V r[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (v + u * kWave < q.tile_vecs) r[u] = load_vec<V, NT>(s + v + u * kWave);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (v + u * kWave < q.tile_vecs) store(v + u * kWave, r[u]);
    }
    return;
  }
  // Small tiles: tile_vecs divides kWave; lane l takes vector l % tile_vecs of
  // tiles a0 + l / tile_vecs, a0 + l / tile_vecs + per_pass, ...
  const int a0 = a * q.group;
  const int tiles = min(q.group, q.n_arrays - a0);
  const int per_pass = kWave / q.tile_vecs;
  const int64_t lane_offset = static_cast<int64_t>(l % q.tile_vecs) * sizeof(V);
  for (int j = l / q.tile_vecs; j < tiles; j += U * per_pass) {
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j + u * per_pass < tiles)
        r[u] = load_vec<V, NT>(as_global<V>(array_base(q.src, a0 + j + u * per_pass) +
                                            src_id * tile_bytes + lane_offset));
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j + u * per_pass < tiles)
        queue_store(as_global<V>(array_base(q.dst, a0 + j + u * per_pass) +
                                 dst_id * tile_bytes + lane_offset), r[u]);
  }
}

// Every wave of the other workgroups is a mover: it takes a claim from its
// cursor, waits for the claim to be published, reads its record, moves its units,
// and counts it finished. Claims hold at most k units each, so they are close in
// size. A claim is taken while the previous one moves, so the atomic's latency
// hides behind the data. Movers are spread over the cursors wave by wave, so the
// claims of a small request land on different compute units.
// Lane 0 runs the claim protocol; the wave's other lanes wait for it (they are
// masked off meanwhile) and take its values with readfirstlane. Nothing is
// shared between the waves of a workgroup, so no barrier is needed: a wave's
// wait for its stores covers all of its lanes.
template <typename V, int U, bool NT>
__device__ void queue_mover(const QueueArgs& q, uint64_t start) {
  const int l = threadIdx.x % kWave;
  QueueState* st = q.state;
  const int cursor = ((blockIdx.x - 1) * (kThreads / kWave) + threadIdx.x / kWave) % kQueueCursors;
  auto take = [&]() -> uint64_t {
    return cursor + kQueueCursors * __hip_atomic_fetch_add(&st->cursor[cursor].left, uint64_t{1},
                                                           __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
  };
  uint64_t next = 0, known = 0, last = start;   // lane 0's
  if (l == 0) next = take();
  for (;;) {
    int32_t go = 0, src = 0, dst = 0, first = 0, end = 0;
    uint32_t desc = 0;
    if (l == 0) {
      const uint64_t claim = next;
      go = wall_clock64() - start <= q.life_ticks ? 1 : 0;
      int nap = 1;
      while (go && claim >= known) {
        const uint64_t pc = agent_word(&st->published_claims);
        if (pc > known) {
          // Sources were written before their descriptor was submitted: lines this
          // CU or XCD cached earlier are dropped before any of them is read. Only
          // a mover whose claim is now published does so: a publication wakes
          // every waiting mover, and thousands of invalidations at once would
          // hold up the few that have work.
          if (claim < pc) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          known = pc;
          last = wall_clock64();
          nap = 1;
          continue;
        }
        if (agent_word(&st->stop)) {
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          const uint64_t final_claims = agent_word(&st->published_claims);
          if (final_claims > known) {
            known = final_claims;
            continue;
          }
          if (claim >= agent_word(&st->stop_claims)) {
            go = 0;
            break;
          }
        }
        if (queue_expired(q, start, last)) {
          go = 0;
          break;
        }
        queue_nap(nap);
        nap = nap < 8 ? 2 * nap : 8;
      }
      if (go) {
        const uint64_t* rec =
            reinterpret_cast<const uint64_t*>(&st->claims[claim % kQueueClaimRing]);
        const uint64_t ids = ring_word(rec), work = ring_word(rec + 1);
        src = static_cast<int32_t>(static_cast<uint32_t>(ids));
        dst = static_cast<int32_t>(static_cast<uint32_t>(ids >> 32));
        first = min(static_cast<int32_t>(work & 0xffff), q.units_per_block);
        end = min(first + static_cast<int32_t>((work >> 16) & 0xffff), q.units_per_block);
        desc = static_cast<uint32_t>(work >> 32);
        next = take();
      }
    }
    if (!__builtin_amdgcn_readfirstlane(go)) return;
    src = __builtin_amdgcn_readfirstlane(src);
    dst = __builtin_amdgcn_readfirstlane(dst);
    end = __builtin_amdgcn_readfirstlane(end);
    for (int u = __builtin_amdgcn_readfirstlane(first); u < end; ++u)
      queue_move_unit<V, U, NT>(q, src, dst, u);
    // The wave's device-coherent stores are complete before the claim counts as
    // finished, and the descriptor's last claim before its completion reaches the host.
    queue_stores_done();
    if (l == 0) {
      const int slot = static_cast<int>(desc % kQueueSlots);
      const uint64_t left = __hip_atomic_fetch_sub(&st->remaining[slot].left, uint64_t{1},
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (left == 1)
        __hip_atomic_store(&q.ring->complete[slot], uint64_t{desc} + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

template <typename V, int U, bool NT>
__global__ void __launch_bounds__(kThreads) kv_queue(QueueArgs q) {
  const uint64_t start = wall_clock64();
  if (blockIdx.x == 0) queue_leader(q, start);
  else queue_mover<V, U, NT>(q, start);
}

using QueueKernel = void (*)(QueueArgs);

template <typename V, bool NT>
QueueKernel queue_kernel_of(int u) {
  if (u >= 8) return kv_queue<V, 8, NT>;
  if (u >= 4) return kv_queue<V, 4, NT>;
  if (u >= 2) return kv_queue<V, 2, NT>;
  return kv_queue<V, 1, NT>;
}

// The queue's kernel for vectors of `vec` bytes, up to lane_vecs of them in
// flight per lane (capped by the unroll setting), as pick_kernel chooses.
QueueKernel pick_queue_kernel(int vec, int lane_vecs, bool nt) {
  const int u = std::min(g_unroll.load(), lane_vecs);
  switch (vec) {
    case 16: return nt ? queue_kernel_of<u32x4, true>(u) : queue_kernel_of<u32x4, false>(u);
    case 8: return kv_queue<u32x2, 4, false>;
    case 4: return kv_queue<uint32_t, 4, false>;
    case 2: return kv_queue<uint16_t, 4, false>;
    default: return kv_queue<uint8_t, 4, false>;
  }
}

}  // namespace

// A request queue: its rings, its stream, and the session the host keeps
// with the kernel (see the protocol at queue_leader).
struct iekv_queue {
  const iekv_pool* src = nullptr;
  const iekv_pool* dst = nullptr;
  bool same_pool = false;
  int32_t workers = 0;              // mover workgroups
  int64_t movers = 0;              // mover waves
  int64_t max_k = 1;               // units per claim at most (claim_bytes)
  int64_t idle_us = 0, life_us = 0;
  QueueRing* ring = nullptr;       // host address of the pinned ring
  QueueState* state = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t ended = nullptr;      // recorded after each launch of the kernel
  QueueKernel kernel = nullptr;
  QueueArgs args{};
  bool running = false;
  bool broken = false;             // a kernel ended with descriptors unfinished
  uint64_t ticket_base = 0;        // ticket of the session's descriptor 0
  uint64_t published = 0;          // descriptors of this session
  uint64_t claims = 0;             // claims of this session
  uint64_t retired = 0;            // descriptors [0, retired) of this session are done
  uint64_t launches = 0;
  std::chrono::steady_clock::time_point started, last_publish;
  std::mutex mu;
};

namespace {

using QueueClock = std::chrono::steady_clock;
constexpr int64_t kQueueWaitUs = 10'000'000;

int64_t us_since(QueueClock::time_point t) {
  return std::chrono::duration_cast<std::chrono::microseconds>(QueueClock::now() - t).count();
}

// Advance q->retired over the descriptors whose completion the kernel wrote.
void queue_retire(iekv_queue* q) {
  while (q->retired < q->published) {
    const uint64_t seen =
        __atomic_load_n(&q->ring->complete[q->retired % kQueueSlots], __ATOMIC_ACQUIRE);
    if (seen < q->retired + 1) break;
    ++q->retired;
  }
}

// Whether the kernel of the current session has ended.
bool queue_ended(iekv_queue* q) {
  const hipError_t e = hipEventQuery(q->ended);
  if (e == hipErrorNotReady) return false;
  if (e != hipSuccess) (void)hipGetLastError();
  return true;
}

int queue_broken() {
  return set_error(IEKV_ERR_HIP, "the queue's kernel ended before finishing its requests; "
                   "the queue cannot be used further");
}

// Start a session: clear both rings' counters and launch the kernel.
int queue_launch(iekv_queue* q) {
  std::memset(static_cast<void*>(q->ring), 0, offsetof(QueueRing, header));
  IEKV_HIP(hipMemsetAsync(q->state, 0, offsetof(QueueState, claims), q->stream));
  q->published = q->claims = q->retired = 0;
  hipLaunchKernelGGL(q->kernel, dim3(static_cast<uint32_t>(q->workers) + 1), dim3(kThreads), 0,
                     q->stream, q->args);
  IEKV_HIP(hipGetLastError());
  IEKV_HIP(hipEventRecord(q->ended, q->stream));
  q->running = true;
  q->started = q->last_publish = QueueClock::now();
  ++q->launches;
  return IEKV_OK;
}

// End the session: the kernel serves every published claim, then exits. The
// wait is bounded by the kernel's own limits (it ends idle_us after its last
// descriptor at the latest).
int queue_end(iekv_queue* q) {
  if (!q->running) return IEKV_OK;
  __atomic_store_n(&q->ring->stop_claims, q->claims, __ATOMIC_RELAXED);
  __atomic_store_n(&q->ring->stop, uint64_t{1}, __ATOMIC_RELEASE);
  const int64_t limit = q->idle_us + kQueueWaitUs;
  const auto t0 = QueueClock::now();
  while (!queue_ended(q)) {
    if (us_since(t0) > limit)
      return set_error(IEKV_ERR_TIMEOUT, "the queue's kernel did not end within %lld us of "
                       "its stop", static_cast<long long>(limit));
    std::this_thread::yield();
  }
  q->running = false;
  queue_retire(q);
  const bool lost = q->retired < q->published;
  q->ticket_base += q->published;
  q->published = q->retired = q->claims = 0;
  if (lost) {
    q->broken = true;
    return queue_broken();
  }
  return IEKV_OK;
}

// Wait (bounded) until the session's descriptors [0, upto] are done.
int queue_wait_local(iekv_queue* q, uint64_t upto, int64_t timeout_us) {
  const auto t0 = QueueClock::now();
  for (uint32_t spin = 0;; ++spin) {
    queue_retire(q);
    if (q->retired > upto) return IEKV_OK;
    if (queue_ended(q)) {
      queue_retire(q);
      if (q->retired > upto) return IEKV_OK;
      q->broken = true;
      return queue_broken();
    }
    if (us_since(t0) > timeout_us)
      return set_error(IEKV_ERR_TIMEOUT, "request %llu not done after %lld us",
                       static_cast<unsigned long long>(q->ticket_base + upto),
                       static_cast<long long>(timeout_us));
    if (spin % 64 == 63) std::this_thread::yield();
    else __builtin_ia32_pause();
  }
}

// Publish one descriptor of n <= kQueueBlocks checked (src, dst) pairs, its
// claims planned for `movers` of the kernel's mover waves (its share of a batch
// submitted together).
int queue_publish(iekv_queue* q, const int32_t* s, const int32_t* d, int32_t n,
                  int64_t movers, uint64_t* ticket) {
  int rc;
  if (q->running && q->published >= kQueueSlots &&
      (rc = queue_wait_local(q, q->published - kQueueSlots, kQueueWaitUs)))
    return rc;
  // A kernel that may end (its idle or lifetime limit) before it sees this
  // descriptor is ended first, and a new one started.
  if (q->running && (us_since(q->last_publish) > q->idle_us / 2 ||
                     us_since(q->started) > q->life_us / 2 || q->published >= (1u << 31)) &&
      (rc = queue_end(q)))
    return rc;
  if (!q->running && (rc = queue_launch(q))) return rc;
  const uint64_t r = q->published;
  const int slot = static_cast<int>(r % kQueueSlots);
  const iekv_plan::QueueClaims c =
      iekv_plan::queue_claims(n, q->args.units_per_block, movers, q->max_k);
  QueueHeader& h = q->ring->header[slot];
  h.claim_base = q->claims;
  h.n_blocks = n;
  h.n_claims = static_cast<int32_t>(c.n_claims);
  h.k = static_cast<int32_t>(c.k);
  h.per_block = static_cast<int32_t>(c.per_block);
  std::memcpy(q->ring->ids[slot], s, sizeof(int32_t) * n);
  std::memcpy(q->ring->ids[slot] + kQueueBlocks, d, sizeof(int32_t) * n);
  __atomic_store_n(&q->ring->tail, r + 1, __ATOMIC_RELEASE);
  q->published = r + 1;
  q->claims += c.n_claims;
  q->last_publish = QueueClock::now();
  *ticket = q->ticket_base + r;
  return IEKV_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------

extern "C" {

int iekv_abi_version(void) { return IEKV_ABI_VERSION; }

const char* iekv_last_error(void) { return g_error.c_str(); }

int iekv_pool_create(const uint64_t* array_ptrs, int32_t n_arrays, int64_t tile_bytes,
                     int64_t num_blocks, int32_t device, iekv_pool** out) {
  if (!out) return set_error(IEKV_ERR_INVALID, "out is null");
  *out = nullptr;
  if (!array_ptrs) return set_error(IEKV_ERR_INVALID, "array_ptrs is null");
  if (n_arrays <= 0 || n_arrays > 65536)
    return set_error(IEKV_ERR_INVALID, "n_arrays %d out of range", n_arrays);
  if (tile_bytes <= 0 || tile_bytes > kMaxTileBytes)
    return set_error(IEKV_ERR_INVALID, "tile_bytes %lld out of range",
                     static_cast<long long>(tile_bytes));
  if (num_blocks <= 0 || num_blocks > INT32_MAX)
    return set_error(IEKV_ERR_INVALID, "num_blocks %lld out of range",
                     static_cast<long long>(num_blocks));
  if (num_blocks > INT64_MAX / tile_bytes)
    return set_error(IEKV_ERR_INVALID, "pool size overflows");
  const int64_t array_bytes = num_blocks * tile_bytes;

  int align = 16;
  while (align > 1 && (tile_bytes % align)) align >>= 1;
  for (int32_t a = 0; a < n_arrays; ++a) {
    if (!array_ptrs[a]) return set_error(IEKV_ERR_INVALID, "array %d address is null", a);
    align = std::min(align, align_of_ptr(array_ptrs[a]));
  }

  // Arrays must not overlap: every byte of every tile belongs to one array.
  std::vector<uint64_t> sorted(array_ptrs, array_ptrs + n_arrays);
  std::sort(sorted.begin(), sorted.end());
  for (int32_t a = 1; a < n_arrays; ++a)
    if (sorted[a] - sorted[a - 1] < static_cast<uint64_t>(array_bytes))
      return set_error(IEKV_ERR_INVALID, "pool arrays overlap (%d arrays of %lld bytes)",
                       n_arrays, static_cast<long long>(array_bytes));

  bool slab = true;
  int64_t stride = array_bytes;
  if (n_arrays > 1) {
    if (array_ptrs[1] <= array_ptrs[0]) {
      slab = false;
    } else {
      stride = static_cast<int64_t>(array_ptrs[1] - array_ptrs[0]);
      for (int32_t a = 2; a < n_arrays && slab; ++a)
        slab = array_ptrs[a] == array_ptrs[0] + static_cast<uint64_t>(a) * stride;
    }
  }

  iekv_pool* p = new (std::nothrow) iekv_pool{};
  if (!p) return set_error(IEKV_ERR_INVALID, "out of host memory");
  p->device = device;
  p->n_arrays = n_arrays;
  p->tile_bytes = tile_bytes;
  p->num_blocks = num_blocks;
  p->align = align;
  p->arrays.assign(array_ptrs, array_ptrs + n_arrays);
  p->lo = sorted.front();
  p->hi = sorted.back() + static_cast<uint64_t>(array_bytes);
  if (slab) {
    p->base = array_ptrs[0];
    p->stride = stride;
  } else {
    DeviceGuard guard(device);
    if (!guard.ok()) {
      delete p;
      return guard.fail();
    }
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->table), sizeof(uint64_t) * n_arrays);
    if (e == hipSuccess)
      e = hipMemcpy(p->table, array_ptrs, sizeof(uint64_t) * n_arrays, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      if (p->table) (void)hipFree(p->table);
      delete p;
      return set_error(IEKV_ERR_HIP, "uploading the pool address table: %s",
                       hipGetErrorString(e));
    }
  }
  *out = p;
  return IEKV_OK;
}

int iekv_pool_destroy(iekv_pool* pool) {
  if (!pool) return IEKV_OK;
  int rc = IEKV_OK;
  if (pool->table) {
    DeviceGuard guard(pool->device);
    hipError_t e = hipFree(pool->table);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      rc = set_error(IEKV_ERR_HIP, "hipFree: %s", hipGetErrorString(e));
    }
  }
  delete pool;
  return rc;
}

int iekv_copy_direct(const iekv_pool* src, const iekv_pool* dst, const int32_t* src_ids,
                     const int32_t* dst_ids, int32_t n_blocks, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_pool(dst, "destination"))) return rc;
  if ((rc = check_ids(src_ids, n_blocks, "source")) ||
      (rc = check_ids(dst_ids, n_blocks, "destination")))
    return rc;
  if (src->n_arrays != dst->n_arrays || src->tile_bytes != dst->tile_bytes)
    return set_error(IEKV_ERR_INVALID,
                     "pools differ in shape: %d arrays x %lld B vs %d arrays x %lld B",
                     src->n_arrays, static_cast<long long>(src->tile_bytes), dst->n_arrays,
                     static_cast<long long>(dst->tile_bytes));
  if (src->device != dst->device)
    return set_error(IEKV_ERR_INVALID, "pools live on devices %d and %d", src->device,
                     dst->device);
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  return launch_move<true, true>(src, dst, nullptr, nullptr, src_ids, dst_ids, n_blocks,
                                 src->tile_bytes, src->n_arrays,
                                 std::min(src->align, dst->align), stream);
}

int iekv_copy_direct_requests(const iekv_pool* src, const iekv_pool* dst, int32_t n_requests,
                              const int32_t* counts, const int32_t* src_ids,
                              const int32_t* dst_ids, const hipStream_t* streams,
                              int32_t n_streams, hipEvent_t* done_events) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_pool(dst, "destination"))) return rc;
  if (n_requests < 0)
    return set_error(IEKV_ERR_INVALID, "n_requests is negative (%d)", n_requests);
  if (n_requests == 0) return IEKV_OK;
  if (!counts) return set_error(IEKV_ERR_INVALID, "counts is null");
  if (n_streams <= 0 || !streams)
    return set_error(IEKV_ERR_INVALID, "need at least one stream (n_streams %d)", n_streams);
  int64_t total = 0;
  for (int32_t k = 0; k < n_requests; ++k) {
    if (counts[k] < 0)
      return set_error(IEKV_ERR_INVALID, "request %d has a negative count (%d)", k, counts[k]);
    total += counts[k];
  }
  if (total > INT32_MAX)
    return set_error(IEKV_ERR_INVALID, "%lld blocks exceed one call", static_cast<long long>(total));
  if ((rc = check_ids(src_ids, static_cast<int32_t>(total), "source")) ||
      (rc = check_ids(dst_ids, static_cast<int32_t>(total), "destination")))
    return rc;
  if (src->n_arrays != dst->n_arrays || src->tile_bytes != dst->tile_bytes)
    return set_error(IEKV_ERR_INVALID, "pools differ in shape");
  if (src->device != dst->device)
    return set_error(IEKV_ERR_INVALID, "pools live on devices %d and %d", src->device,
                     dst->device);
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  const int align = std::min(src->align, dst->align);
  int64_t at = 0;
  for (int32_t k = 0; k < n_requests; ++k) {
    hipStream_t stream = streams[k % n_streams];
    if ((rc = launch_move<true, true>(src, dst, nullptr, nullptr, src_ids + at, dst_ids + at,
                                      counts[k], src->tile_bytes, src->n_arrays, align, stream)))
      return rc;
    if (done_events) IEKV_HIP(hipEventRecord(done_events[k], stream));
    at += counts[k];
  }
  return IEKV_OK;
}

int iekv_pack(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks, void* staging,
              int64_t staging_bytes, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_ids(src_ids, n_blocks, "source")))
    return rc;
  const int64_t need = image_bytes(src, n_blocks);
  if (need < 0) return set_error(IEKV_ERR_INVALID, "staging size overflows");
  if ((rc = check_buffer(staging, staging_bytes, need, "staging"))) return rc;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  const int align = std::min(src->align, align_of_ptr(reinterpret_cast<uint64_t>(staging)));
  return launch_move<true, false>(src, nullptr, nullptr, static_cast<char*>(staging), src_ids,
                                  nullptr, n_blocks, src->tile_bytes, src->n_arrays, align,
                                  stream);
}

int iekv_unpack(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                const void* staging, int64_t staging_bytes, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(dst, "destination")) ||
      (rc = check_ids(dst_ids, n_blocks, "destination")))
    return rc;
  const int64_t need = image_bytes(dst, n_blocks);
  if (need < 0) return set_error(IEKV_ERR_INVALID, "staging size overflows");
  if ((rc = check_buffer(staging, staging_bytes, need, "staging"))) return rc;
  DeviceGuard guard(dst->device);
  if (!guard.ok()) return guard.fail();
  const int align = std::min(dst->align, align_of_ptr(reinterpret_cast<uint64_t>(staging)));
  return launch_move<false, true>(nullptr, dst, static_cast<const char*>(staging), nullptr,
                                  nullptr, dst_ids, n_blocks, dst->tile_bytes, dst->n_arrays,
                                  align, stream);
}

int iekv_copy_direct_ids(const iekv_pool* src, const iekv_pool* dst, const int32_t* src_ids,
                         const int32_t* dst_ids, int32_t n_blocks, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_pool(dst, "destination")) ||
      (rc = check_host_count(n_blocks, src_ids, dst_ids)))
    return rc;
  if (src->n_arrays != dst->n_arrays || src->tile_bytes != dst->tile_bytes)
    return set_error(IEKV_ERR_INVALID, "pools differ in shape");
  if (src->device != dst->device)
    return set_error(IEKV_ERR_INVALID, "pools live on devices %d and %d", src->device,
                     dst->device);
  std::vector<int32_t> s, d;
  bool same_pool = false;
  if ((rc = check_aliasing(src, dst, &same_pool)) ||
      (rc = check_host_range(src_ids, n_blocks, src->num_blocks, "source")) ||
      (rc = check_host_range(dst_ids, n_blocks, dst->num_blocks, "destination")) ||
      (rc = order_pairs(src_ids, dst_ids, n_blocks, same_pool, &s, &d)))
    return rc;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  return launch_host_ids<true, true>(src, dst, nullptr, nullptr, s.data(), d.data(), n_blocks,
                                     src->tile_bytes, src->n_arrays,
                                     std::min(src->align, dst->align), stream);
}

int iekv_pack_ids(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks, void* staging,
                  int64_t staging_bytes, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_host_count(n_blocks, src_ids, src_ids)))
    return rc;
  const int64_t need = image_bytes(src, n_blocks);
  if (need < 0) return set_error(IEKV_ERR_INVALID, "staging size overflows");
  if ((rc = check_buffer(staging, staging_bytes, need, "staging"))) return rc;
  if ((rc = check_host_range(src_ids, n_blocks, src->num_blocks, "source"))) return rc;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  const int align = std::min(src->align, align_of_ptr(reinterpret_cast<uint64_t>(staging)));
  return launch_host_ids<true, false>(src, nullptr, nullptr, static_cast<char*>(staging), src_ids,
                                      nullptr, n_blocks, src->tile_bytes, src->n_arrays, align,
                                      stream);
}

int iekv_unpack_ids(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                    const void* staging, int64_t staging_bytes, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(dst, "destination")) ||
      (rc = check_host_count(n_blocks, dst_ids, dst_ids)))
    return rc;
  const int64_t need = image_bytes(dst, n_blocks);
  if (need < 0) return set_error(IEKV_ERR_INVALID, "staging size overflows");
  if ((rc = check_buffer(staging, staging_bytes, need, "staging"))) return rc;
  if ((rc = check_host_range(dst_ids, n_blocks, dst->num_blocks, "destination")) ||
      (rc = check_distinct(dst_ids, n_blocks, "destination")))
    return rc;
  DeviceGuard guard(dst->device);
  if (!guard.ok()) return guard.fail();
  const int align = std::min(dst->align, align_of_ptr(reinterpret_cast<uint64_t>(staging)));
  return launch_host_ids<false, true>(nullptr, dst, static_cast<const char*>(staging), nullptr,
                                      nullptr, dst_ids, n_blocks, dst->tile_bytes, dst->n_arrays,
                                      align, stream);
}

int iekv_write_slots_layers(const iekv_pool* pool, int32_t first_layer, int32_t n_layers,
                            int32_t block_size, const void* k, const void* v,
                            int64_t layer_stride, const int64_t* slots, int32_t n_tokens,
                            hipStream_t stream) {
  int rc;
  if ((rc = check_pool(pool, "destination"))) return rc;
  const int32_t layers = pool->n_arrays / 2;
  if (pool->n_arrays % 2 || first_layer < 0 || n_layers <= 0 ||
      first_layer > layers - n_layers)
    return set_error(IEKV_ERR_INVALID, "layers %d..%d out of range for %d layers", first_layer,
                     first_layer + n_layers - 1, layers);
  if (block_size <= 0 || pool->tile_bytes % block_size)
    return set_error(IEKV_ERR_INVALID, "block_size %d does not divide the %lld-byte tile",
                     block_size, static_cast<long long>(pool->tile_bytes));
  if (layer_stride < 0)
    return set_error(IEKV_ERR_INVALID, "layer_stride is negative (%lld)",
                     static_cast<long long>(layer_stride));
  if (n_tokens < 0) return set_error(IEKV_ERR_INVALID, "n_tokens is negative (%d)", n_tokens);
  if (n_tokens == 0) return IEKV_OK;
  if (!k || !v || !slots) return set_error(IEKV_ERR_INVALID, "k, v or slots is null");
  const int64_t row_bytes = pool->tile_bytes / block_size;
  const int align = std::min(row_align(row_bytes, pool->align, {k, v}),
                             layer_stride ? align_of_ptr(static_cast<uint64_t>(layer_stride))
                                          : 16);
  RowShape sh;
  uint32_t grid = 0;
  const int vec = align >= 16 ? 16 : align;
  if (!row_shape(row_bytes, vec, n_tokens, 2 * n_layers,
                 (g_order.load() & iekv_plan::kXcdGrouped) != 0, &sh, &grid))
    return set_error(IEKV_ERR_INVALID, "%d tokens in %d layers exceed one launch", n_tokens,
                     n_layers);
  DeviceGuard guard(pool->device);
  if (!guard.ok()) return guard.fail();
  const int64_t pool_rows = pool->num_blocks * block_size;
  const char* kc = static_cast<const char*>(k);
  const char* vc = static_cast<const char*>(v);
  const PoolView view = view_of(pool);
  const bool nt = g_nontemporal.load() != 0;
  constexpr bool kNts = IEKV_SCATTER_NT_STORES != 0;
#define IEKV_SCATTER(T)                                                                      \
  (nt ? dispatch(kv_scatter_rows<T, true, kNts>, dim3(grid), stream, view, layers,          \
                 first_layer, n_layers, kc, vc, layer_stride, slots, n_tokens, sh, pool_rows) \
      : dispatch(kv_scatter_rows<T, false, false>, dim3(grid), stream, view, layers,         \
                 first_layer, n_layers, kc, vc, layer_stride, slots, n_tokens, sh, pool_rows))
  if (vec >= 16) return IEKV_SCATTER(u32x4);
  if (vec >= 8) return IEKV_SCATTER(u32x2);
  if (vec >= 4) return IEKV_SCATTER(uint32_t);
  if (vec >= 2) return IEKV_SCATTER(uint16_t);
  return IEKV_SCATTER(uint8_t);
#undef IEKV_SCATTER
}

int iekv_write_slots(const iekv_pool* pool, int32_t layer, int32_t block_size, const void* k,
                     const void* v, const int64_t* slots, int32_t n_tokens, hipStream_t stream) {
  return iekv_write_slots_layers(pool, layer, 1, block_size, k, v, 0, slots, n_tokens, stream);
}

int iekv_gather_rows_arrays(const iekv_pool* pool, int32_t first_array, int32_t n_arrays,
                            int32_t block_size, const int32_t* block_table, int32_t context_len,
                            void* out, int64_t out_bytes, hipStream_t stream) {
  int rc;
  if ((rc = check_pool(pool, "source"))) return rc;
  if (first_array < 0 || n_arrays <= 0 || first_array > pool->n_arrays - n_arrays)
    return set_error(IEKV_ERR_INVALID, "arrays %d..%d out of range for %d arrays", first_array,
                     first_array + n_arrays - 1, pool->n_arrays);
  if (block_size <= 0 || pool->tile_bytes % block_size)
    return set_error(IEKV_ERR_INVALID, "block_size %d does not divide the %lld-byte tile",
                     block_size, static_cast<long long>(pool->tile_bytes));
  if (context_len < 0)
    return set_error(IEKV_ERR_INVALID, "context_len is negative (%d)", context_len);
  if (context_len == 0) return IEKV_OK;
  const int64_t row_bytes = pool->tile_bytes / block_size;
  const int64_t out_stride = row_bytes * context_len;
  if (n_arrays > 1 && out_stride > INT64_MAX / n_arrays)
    return set_error(IEKV_ERR_INVALID, "output size overflows");
  if ((rc = check_buffer(out, out_bytes, out_stride * n_arrays, "output"))) return rc;
  if (!block_table) return set_error(IEKV_ERR_INVALID, "block_table is null");
  const int align = row_align(row_bytes, pool->align, {out});
  const int vec = align >= 16 ? 16 : align;
  RowShape sh;
  uint32_t grid = 0;
  if (!row_shape(row_bytes, vec, context_len, n_arrays,
                 (g_pack_order.load() & iekv_plan::kXcdGrouped) != 0, &sh, &grid))
    return set_error(IEKV_ERR_INVALID, "a context of %d rows in %d arrays exceeds one launch",
                     context_len, n_arrays);
  DeviceGuard guard(pool->device);
  if (!guard.ok()) return guard.fail();
  char* oc = static_cast<char*>(out);
  const PoolView view = view_of(pool);
  const bool nt = g_nontemporal.load() != 0;
#define IEKV_GATHER(T)                                                                      \
  (nt ? dispatch(kv_gather_rows<T, true, true>, dim3(grid), stream, view, first_array,      \
                 block_table, block_size, oc, out_stride, context_len, sh)                  \
      : dispatch(kv_gather_rows<T, false, false>, dim3(grid), stream, view, first_array,    \
                 block_table, block_size, oc, out_stride, context_len, sh))
  if (vec >= 16) return IEKV_GATHER(u32x4);
  if (vec >= 8) return IEKV_GATHER(u32x2);
  if (vec >= 4) return IEKV_GATHER(uint32_t);
  if (vec >= 2) return IEKV_GATHER(uint16_t);
  return IEKV_GATHER(uint8_t);
#undef IEKV_GATHER
}

int iekv_gather_rows(const iekv_pool* pool, int32_t array, int32_t block_size,
                     const int32_t* block_table, int32_t context_len, void* out,
                     int64_t out_bytes, hipStream_t stream) {
  return iekv_gather_rows_arrays(pool, array, 1, block_size, block_table, context_len, out,
                                 out_bytes, stream);
}

int iekv_offload(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                 void* host_dst, int64_t host_bytes, void* staging, int64_t staging_bytes,
                 hipStream_t compute, hipStream_t copy) {
  int rc;
  int64_t need = 0;
  if ((rc = check_offload(src, src_ids, n_blocks, host_dst, host_bytes, &need))) return rc;
  if (n_blocks == 0) return IEKV_OK;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  return run_offload(src, {src_ids, false}, n_blocks, host_dst, need,
                     static_cast<char*>(staging), staging_bytes, compute, copy, nullptr);
}

int iekv_offload_ids(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                     void* host_dst, int64_t host_bytes, void* staging, int64_t staging_bytes,
                     hipStream_t compute, hipStream_t copy) {
  int rc;
  int64_t need = 0;
  if ((rc = check_offload(src, src_ids, n_blocks, host_dst, host_bytes, &need)) ||
      (rc = check_host_range(src_ids, n_blocks, src->num_blocks, "source")))
    return rc;
  if (n_blocks == 0) return IEKV_OK;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  return run_offload(src, {src_ids, true}, n_blocks, host_dst, need,
                     static_cast<char*>(staging), staging_bytes, compute, copy, nullptr);
}

int iekv_offload_static(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                        void* host_dst, int64_t host_bytes, hipStream_t compute,
                        hipStream_t copy) {
  int rc;
  int64_t need = 0;
  if ((rc = check_offload(src, src_ids, n_blocks, host_dst, host_bytes, &need))) return rc;
  const int64_t block_bytes = image_bytes(src, 1);
  if (block_bytes > IEKV_STATIC_STAGING_BYTES)
    return set_error(IEKV_ERR_CAPACITY,
                     "a block image of %lld bytes exceeds the %lld-byte static staging buffer; "
                     "use iekv_offload with a staging buffer of at least one block image",
                     static_cast<long long>(block_bytes),
                     static_cast<long long>(IEKV_STATIC_STAGING_BYTES));
  if (n_blocks == 0) return IEKV_OK;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  std::lock_guard<std::mutex> lock(g_static_mu);
  StaticStaging* st = nullptr;
  if ((rc = static_staging(src->device, &st))) return rc;
  return run_offload(src, {src_ids, false}, n_blocks, host_dst, need, st->ptr,
                     IEKV_STATIC_STAGING_BYTES, compute, copy, &st->events);
}

int iekv_restore(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                 const void* host_src, int64_t host_bytes, void* staging, int64_t staging_bytes,
                 hipStream_t compute, hipStream_t copy) {
  int rc;
  if ((rc = check_pool(dst, "destination")) ||
      (rc = check_ids(dst_ids, n_blocks, "destination")))
    return rc;
  return restore_image(dst, {dst_ids, false}, n_blocks, host_src, host_bytes, staging,
                       staging_bytes, compute, copy);
}

int iekv_restore_ids(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                     const void* host_src, int64_t host_bytes, void* staging,
                     int64_t staging_bytes, hipStream_t compute, hipStream_t copy) {
  int rc;
  if ((rc = check_pool(dst, "destination")) ||
      (rc = check_ids(dst_ids, n_blocks, "destination")) ||
      (rc = check_host_range(dst_ids, n_blocks, dst->num_blocks, "destination")) ||
      (rc = check_distinct(dst_ids, n_blocks, "destination")))
    return rc;
  return restore_image(dst, {dst_ids, true}, n_blocks, host_src, host_bytes, staging,
                       staging_bytes, compute, copy);
}

int iekv_restore_blocks(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                        const void* const* host_blocks, void* staging, int64_t staging_bytes,
                        hipStream_t compute, hipStream_t copy) {
  int rc;
  if ((rc = check_pool(dst, "destination")) ||
      (rc = check_ids(dst_ids, n_blocks, "destination")))
    return rc;
  return restore_images(dst, {dst_ids, false}, n_blocks, host_blocks, staging, staging_bytes,
                        compute, copy);
}

int iekv_restore_blocks_ids(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                            const void* const* host_blocks, void* staging,
                            int64_t staging_bytes, hipStream_t compute, hipStream_t copy) {
  int rc;
  if ((rc = check_pool(dst, "destination")) ||
      (rc = check_ids(dst_ids, n_blocks, "destination")) ||
      (rc = check_host_range(dst_ids, n_blocks, dst->num_blocks, "destination")) ||
      (rc = check_distinct(dst_ids, n_blocks, "destination")))
    return rc;
  return restore_images(dst, {dst_ids, true}, n_blocks, host_blocks, staging, staging_bytes,
                        compute, copy);
}

int iekv_offload_blocks(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                        void* const* host_blocks, void* staging, int64_t staging_bytes,
                        hipStream_t compute, hipStream_t copy) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_ids(src_ids, n_blocks, "source")))
    return rc;
  return offload_images(src, {src_ids, false}, n_blocks, host_blocks, staging, staging_bytes,
                        compute, copy);
}

int iekv_offload_blocks_ids(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                            void* const* host_blocks, void* staging, int64_t staging_bytes,
                            hipStream_t compute, hipStream_t copy) {
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_ids(src_ids, n_blocks, "source")) ||
      (rc = check_host_range(src_ids, n_blocks, src->num_blocks, "source")))
    return rc;
  return offload_images(src, {src_ids, true}, n_blocks, host_blocks, staging, staging_bytes,
                        compute, copy);
}

int iekv_check_ids(const iekv_pool* src, const int32_t* src_ids, const iekv_pool* dst,
                   const int32_t* dst_ids, int32_t n_blocks, void* workspace,
                   int64_t workspace_bytes, int32_t* status, hipStream_t stream) {
  int rc;
  if (!src && !dst) return set_error(IEKV_ERR_INVALID, "no source or destination pool");
  if (src && (rc = check_ids(src_ids, n_blocks, "source"))) return rc;
  if (dst && (rc = check_ids(dst_ids, n_blocks, "destination"))) return rc;
  if (!status) return set_error(IEKV_ERR_INVALID, "status is null");
  if (reinterpret_cast<uintptr_t>(status) % alignof(int32_t))
    return set_error(IEKV_ERR_INVALID, "status is not 4-byte aligned");
  if (src && dst && src->device != dst->device)
    return set_error(IEKV_ERR_INVALID, "pools live on devices %d and %d", src->device,
                     dst->device);
  bool same_pool = false;
  if (src && dst && (rc = check_aliasing(src, dst, &same_pool))) return rc;
  const int64_t words = dst ? (dst->num_blocks + 31) / 32 : 0;
  if ((rc = check_buffer(workspace, workspace_bytes, words * 4, "workspace"))) return rc;
  if (words && reinterpret_cast<uintptr_t>(workspace) % alignof(uint32_t))
    return set_error(IEKV_ERR_INVALID, "workspace is not 4-byte aligned");
  DeviceGuard guard((src ? src : dst)->device);
  if (!guard.ok()) return guard.fail();
  auto* bitmap = static_cast<uint32_t*>(workspace);
  const uint32_t clear_grid =
      static_cast<uint32_t>(std::clamp<int64_t>((words + kThreads - 1) / kThreads, 1, 4096));
  hipLaunchKernelGGL(ids_clear, dim3(clear_grid), dim3(kThreads), 0, stream, bitmap, words,
                     status, static_cast<int32_t>(clear_grid));
  IEKV_HIP(hipGetLastError());
  if (n_blocks == 0) return IEKV_OK;
  const uint32_t grid = static_cast<uint32_t>((static_cast<int64_t>(n_blocks) + kThreads - 1) /
                                              kThreads);
  if (dst) {
    hipLaunchKernelGGL(ids_mark, dim3(grid), dim3(kThreads), 0, stream, dst_ids, n_blocks,
                       dst->num_blocks, bitmap, status);
    IEKV_HIP(hipGetLastError());
  }
  if (src) {
    hipLaunchKernelGGL(ids_probe, dim3(grid), dim3(kThreads), 0, stream, src_ids, n_blocks,
                       src->num_blocks, same_pool ? static_cast<const uint32_t*>(bitmap)
                                                  : nullptr, status);
    IEKV_HIP(hipGetLastError());
  }
  return IEKV_OK;
}

int iekv_noop(int32_t workgroups, int32_t launches, hipStream_t stream) {
  if (workgroups <= 0 || workgroups > kMaxGrid)
    return set_error(IEKV_ERR_INVALID, "workgroups %d out of range", workgroups);
  if (launches < 0) return set_error(IEKV_ERR_INVALID, "launches is negative (%d)", launches);
  for (int32_t i = 0; i < launches; ++i) {
    const int rc = dispatch(kv_noop, dim3(static_cast<uint32_t>(workgroups)), stream);
    if (rc) return rc;
  }
  return IEKV_OK;
}

int iekv_host_alloc(int64_t bytes, void** out) {
  if (!out) return set_error(IEKV_ERR_INVALID, "out is null");
  *out = nullptr;
  if (bytes <= 0) return set_error(IEKV_ERR_INVALID, "bytes must be positive (%lld)",
                                   static_cast<long long>(bytes));
  const hipError_t e = hipHostMalloc(out, static_cast<size_t>(bytes), hipHostMallocDefault);
  if (e != hipSuccess || !*out) {
    (void)hipGetLastError();
    *out = nullptr;
    return set_error(IEKV_ERR_HIP, "hipHostMalloc of %lld bytes: %s",
                     static_cast<long long>(bytes),
                     e != hipSuccess ? hipGetErrorString(e) : "null pointer");
  }
  return IEKV_OK;
}

int iekv_host_free(void* ptr) {
  if (!ptr) return IEKV_OK;
  IEKV_HIP(hipHostFree(ptr));
  return IEKV_OK;
}

int iekv_profile_start(int32_t max_launches) {
  if (max_launches <= 0 || max_launches > (1 << 20))
    return set_error(IEKV_ERR_INVALID, "max_launches %d out of range", max_launches);
  Profiler& prof = g_profiler;
  int device = 0;
  IEKV_HIP(hipGetDevice(&device));
  if (prof.device != device) {
    prof.release();
    prof.device = device;
  }
  while (prof.events.size() < static_cast<size_t>(max_launches)) {
    hipEvent_t a = nullptr, b = nullptr;
    IEKV_HIP(hipEventCreate(&a));
    hipError_t e = hipEventCreate(&b);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      (void)hipEventDestroy(a);
      return set_error(IEKV_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(e));
    }
    prof.events.emplace_back(a, b);
  }
  prof.used = 0;
  prof.on = true;
  return IEKV_OK;
}

int iekv_profile_stop(float* durations_ms, int32_t capacity, int32_t* count) {
  Profiler& prof = g_profiler;
  const size_t n = prof.on ? prof.used : 0;
  prof.on = false;
  prof.used = 0;
  if (count) *count = static_cast<int32_t>(n);
  if (n == 0) return IEKV_OK;
  IEKV_HIP(hipEventSynchronize(prof.events[n - 1].second));
  const size_t m = durations_ms ? std::min<size_t>(n, capacity > 0 ? capacity : 0) : 0;
  for (size_t i = 0; i < m; ++i) {
    IEKV_HIP(hipEventSynchronize(prof.events[i].second));
    IEKV_HIP(hipEventElapsedTime(&durations_ms[i], prof.events[i].first,
                                 prof.events[i].second));
  }
  return IEKV_OK;
}

int iekv_set_launch(int32_t run_blocks, int32_t unroll, int32_t nontemporal, int32_t order,
                    int32_t pack_order, int32_t chunk_bytes) {
  if (run_blocks < -1 || run_blocks > kMaxRun)
    return set_error(IEKV_ERR_INVALID, "run_blocks %d out of range", run_blocks);
  if (unroll != 0 && unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16)
    return set_error(IEKV_ERR_INVALID, "unroll must be 1, 2, 4, 8 or 16 (got %d)", unroll);
  if (nontemporal < -1 || nontemporal > 1)
    return set_error(IEKV_ERR_INVALID, "nontemporal must be -1, 0 or 1 (got %d)", nontemporal);
  if (!valid_order(order))
    return set_error(IEKV_ERR_INVALID, "order must be -1 or 0..7 (got %d)", order);
  if (!valid_order(pack_order))
    return set_error(IEKV_ERR_INVALID, "pack_order must be -1 or 0..7 (got %d)",
                     pack_order);
  if (!valid_chunk(chunk_bytes))
    return set_error(IEKV_ERR_INVALID,
                     "chunk_bytes must be -1, 0 or a power of two from 64 to 1 MiB (got %d)",
                     chunk_bytes);
  if (run_blocks >= 0) g_run.store(run_blocks);
  if (unroll) g_unroll.store(unroll);
  if (nontemporal >= 0) g_nontemporal.store(nontemporal);
  if (order >= 0) g_order.store(order);
  if (pack_order >= 0) g_pack_order.store(pack_order);
  if (chunk_bytes >= 0) {
    g_chunk.store(chunk_bytes);
    g_direct_chunk.store(chunk_bytes);
  }
  return IEKV_OK;
}

int iekv_set_direct_chunk(int32_t chunk_bytes) {
  if (!valid_chunk(chunk_bytes))
    return set_error(IEKV_ERR_INVALID,
                     "chunk_bytes must be -1, 0 or a power of two from 64 to 1 MiB (got %d)",
                     chunk_bytes);
  if (chunk_bytes >= 0) g_direct_chunk.store(chunk_bytes);
  return IEKV_OK;
}

int iekv_get_direct_chunk(int32_t* chunk_bytes) {
  if (!chunk_bytes) return set_error(IEKV_ERR_INVALID, "null output pointer");
  *chunk_bytes = g_direct_chunk.load();
  return IEKV_OK;
}

int iekv_get_launch(int32_t* run_blocks, int32_t* unroll, int32_t* nontemporal,
                    int32_t* order, int32_t* pack_order, int32_t* chunk_bytes) {
  if (run_blocks) *run_blocks = g_run.load();
  if (unroll) *unroll = g_unroll.load();
  if (nontemporal) *nontemporal = g_nontemporal.load();
  if (order) *order = g_order.load();
  if (pack_order) *pack_order = g_pack_order.load();
  if (chunk_bytes) *chunk_bytes = g_chunk.load();
  return IEKV_OK;
}

int iekv_queue_create(const iekv_pool* src, const iekv_pool* dst, int32_t workers,
                      int64_t claim_bytes, int64_t idle_us, int64_t life_us, iekv_queue** out) {
  if (!out) return set_error(IEKV_ERR_INVALID, "out is null");
  *out = nullptr;
  int rc;
  if ((rc = check_pool(src, "source")) || (rc = check_pool(dst, "destination"))) return rc;
  if (src->n_arrays != dst->n_arrays || src->tile_bytes != dst->tile_bytes)
    return set_error(IEKV_ERR_INVALID, "pools differ in shape");
  if (src->device != dst->device)
    return set_error(IEKV_ERR_INVALID, "pools live on devices %d and %d", src->device,
                     dst->device);
  bool same_pool = false;
  if ((rc = check_aliasing(src, dst, &same_pool))) return rc;
  if (workers < 0 || claim_bytes < 0 || idle_us < 0 || life_us < 0)
    return set_error(IEKV_ERR_INVALID, "negative queue setting");
  if (idle_us == 0) idle_us = 200'000;
  if (life_us == 0) life_us = 60'000'000;
  if (idle_us < 1000 || idle_us > 60'000'000 || life_us < 2 * idle_us || life_us > 3'600'000'000LL)
    return set_error(IEKV_ERR_INVALID, "idle_us %lld / life_us %lld out of range (idle 1 ms to "
                     "60 s, life at least twice idle and at most 1 h)",
                     static_cast<long long>(idle_us), static_cast<long long>(life_us));
  // 512 KiB claims: large requests 6.19 TB/s against 6.11 with 128 KiB (cfg3); small
  // requests' claims are bounded by their blocks and their share of the movers.
  if (claim_bytes == 0) claim_bytes = 512 << 10;
  DeviceGuard guard(src->device);
  if (!guard.ok()) return guard.fail();
  int cus = 0, clock_khz = 0;
  IEKV_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, src->device));
  IEKV_HIP(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, src->device));
  if (clock_khz <= 0) return set_error(IEKV_ERR_HIP, "the device reports no wall clock");
  if (workers > 65535) return set_error(IEKV_ERR_INVALID, "workers %d out of range", workers);

  // The unit of work: one tile, or a group of small tiles of one block, as the
  // pool-to-pool launches move them (plan_move with the pool-writing chunk).
  MovePlan pl;
  const int align = std::min(src->align, dst->align);
  if ((rc = plan_move(1, src->tile_bytes, src->n_arrays, align, true, true, true, &pl,
                      g_direct_chunk.load())))
    return rc;
  // A unit is a whole tile, or a group of small tiles, moved by one wave.
  const int group = iekv_plan::queue_tile_group(pl.tile_vecs, pl.vec, g_direct_chunk.load(),
                                                src->n_arrays);
  const int64_t lane_vecs = (static_cast<int64_t>(pl.tile_vecs) * group + kWave - 1) / kWave;
  const int64_t unit_bytes = src->tile_bytes * group;
  const int32_t units_per_block = (src->n_arrays + group - 1) / group;
  if (units_per_block > kQueueMaxUnits)
    return set_error(IEKV_ERR_INVALID, "%d units per block exceed the queue's %d",
                     units_per_block, kQueueMaxUnits);

  iekv_queue* q = new (std::nothrow) iekv_queue{};
  if (!q) return set_error(IEKV_ERR_INVALID, "out of host memory");
  auto fail = [&](int code) {
    if (q->ended) (void)hipEventDestroy(q->ended);
    if (q->stream) (void)hipStreamDestroy(q->stream);
    if (q->state) (void)hipFree(q->state);
    if (q->ring) (void)hipHostFree(q->ring);
    delete q;
    return code;
  };
#define IEKV_QUEUE_HIP(expr)                                                                  \
  do {                                                                                        \
    const hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess) {                                                                   \
      (void)hipGetLastError();                                                                \
      return fail(set_error(IEKV_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)));           \
    }                                                                                         \
  } while (0)
  IEKV_QUEUE_HIP(hipHostMalloc(reinterpret_cast<void**>(&q->ring), sizeof(QueueRing),
                               hipHostMallocCoherent | hipHostMallocMapped));
  std::memset(static_cast<void*>(q->ring), 0, sizeof(QueueRing));
  void* ring_dev = nullptr;
  IEKV_QUEUE_HIP(hipHostGetDevicePointer(&ring_dev, q->ring, 0));
  IEKV_QUEUE_HIP(hipMalloc(reinterpret_cast<void**>(&q->state), sizeof(QueueState)));
  IEKV_QUEUE_HIP(hipMemset(q->state, 0, sizeof(QueueState)));
  // Non-blocking: work on the legacy default stream must not wait for the
  // resident kernel.
  IEKV_QUEUE_HIP(hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking));
  IEKV_QUEUE_HIP(hipEventCreateWithFlags(&q->ended, hipEventDisableTiming));
  IEKV_QUEUE_HIP(hipEventRecord(q->ended, q->stream));
#undef IEKV_QUEUE_HIP
  q->src = src;
  q->dst = dst;
  q->same_pool = same_pool;
  q->workers = workers;
  q->movers = workers * (kThreads / kWave);
  q->max_k = std::max<int64_t>(1, claim_bytes / unit_bytes);
  q->idle_us = idle_us;
  q->life_us = life_us;
  q->kernel = pick_queue_kernel(pl.vec, static_cast<int>(std::min<int64_t>(lane_vecs, 16)),
                                nontemporal(-1));
  if (workers == 0) {
    // One workgroup per compute unit, the leader's included (4 mover waves per CU).
    // Measured on MI355X against 2 per CU and up to the 4 that fit: a step of 64
    // small requests 0.054 ms against 0.063 and 0.080 (cfg1), large requests 6.25
    // against 6.21 and 6.19 TB/s (cfg3); cfg2's 1.5-block requests 6% slower than with
    // 2. It also leaves the other kernels of a serving step most of the GPU.
    workers = std::max(1, cus - 1);
    q->workers = workers;
    q->movers = static_cast<int64_t>(workers) * (kThreads / kWave);
  }
  const uint64_t ticks_per_us = static_cast<uint64_t>(clock_khz) / 1000;
  q->args = QueueArgs{view_of(src), view_of(dst), q->state, static_cast<QueueRing*>(ring_dev),
                      pl.tile_vecs, src->n_arrays, group, units_per_block,
                      static_cast<uint64_t>(idle_us) * std::max<uint64_t>(ticks_per_us, 1),
                      static_cast<uint64_t>(life_us) * std::max<uint64_t>(ticks_per_us, 1)};
  *out = q;
  return IEKV_OK;
}

int iekv_queue_submit(iekv_queue* q, const int32_t* src_ids, const int32_t* dst_ids,
                      int32_t n_blocks, uint64_t* ticket) {
  if (!ticket) return set_error(IEKV_ERR_INVALID, "ticket is null");
  return iekv_queue_submit_requests(q, 1, &n_blocks, src_ids, dst_ids, ticket);
}

int iekv_queue_submit_requests(iekv_queue* q, int32_t n_requests, const int32_t* counts,
                               const int32_t* src_ids, const int32_t* dst_ids,
                               uint64_t* tickets) {
  if (!q) return set_error(IEKV_ERR_INVALID, "queue is null");
  if (n_requests < 0)
    return set_error(IEKV_ERR_INVALID, "n_requests is negative (%d)", n_requests);
  if (n_requests == 0) return IEKV_OK;
  if (!counts || !tickets) return set_error(IEKV_ERR_INVALID, "counts or tickets is null");
  int64_t total = 0;
  for (int32_t k = 0; k < n_requests; ++k) {
    if (counts[k] < 0)
      return set_error(IEKV_ERR_INVALID, "request %d has a negative count (%d)", k, counts[k]);
    total += counts[k];
  }
  if (total > INT32_MAX)
    return set_error(IEKV_ERR_INVALID, "%lld blocks exceed one call",
                     static_cast<long long>(total));
  int rc;
  if ((rc = check_host_count(static_cast<int32_t>(total), src_ids, dst_ids))) return rc;
  // Every request is checked before any is published.
  std::vector<int32_t> s(static_cast<size_t>(total)), d(static_cast<size_t>(total));
  std::vector<int32_t> rs, rd;
  for (int64_t k = 0, at = 0; k < n_requests; at += counts[k], ++k) {
    const int32_t n = counts[k];
    if ((rc = check_host_range(src_ids + at, n, q->src->num_blocks, "source")) ||
        (rc = check_host_range(dst_ids + at, n, q->dst->num_blocks, "destination")) ||
        (rc = order_pairs(src_ids + at, dst_ids + at, n, q->same_pool, &rs, &rd)))
      return rc;
    std::copy(rs.begin(), rs.end(), s.begin() + at);
    std::copy(rd.begin(), rd.end(), d.begin() + at);
  }
  std::lock_guard<std::mutex> lock(q->mu);
  if (q->broken) return queue_broken();
  DeviceGuard guard(q->src->device);
  if (!guard.ok()) return guard.fail();
  // The batch's units are spread over every mover: a descriptor's claims are
  // planned for its share of them.
  for (int64_t k = 0, at = 0; k < n_requests; at += counts[k], ++k) {
    tickets[k] = IEKV_QUEUE_DONE;
    for (int32_t first = 0; first < counts[k]; first += kQueueBlocks) {
      const int32_t m = std::min<int32_t>(kQueueBlocks, counts[k] - first);
      const int64_t share = std::max<int64_t>(1, q->movers * m / total);
      if ((rc = queue_publish(q, s.data() + at + first, d.data() + at + first, m, share,
                              &tickets[k])))
        return rc;
    }
  }
  return IEKV_OK;
}

int iekv_queue_wait(iekv_queue* q, uint64_t ticket, int64_t timeout_us) {
  if (!q) return set_error(IEKV_ERR_INVALID, "queue is null");
  if (ticket == IEKV_QUEUE_DONE) return IEKV_OK;
  std::lock_guard<std::mutex> lock(q->mu);
  if (q->broken) return queue_broken();
  if (ticket >= q->ticket_base + q->published)
    return set_error(IEKV_ERR_INVALID, "ticket %llu was not issued",
                     static_cast<unsigned long long>(ticket));
  if (ticket < q->ticket_base) return IEKV_OK;   // an ended session served all of its own
  return queue_wait_local(q, ticket - q->ticket_base, timeout_us < 0 ? kQueueWaitUs : timeout_us);
}

int iekv_queue_poll(iekv_queue* q, uint64_t ticket, int32_t* done) {
  if (!q || !done) return set_error(IEKV_ERR_INVALID, "queue or done is null");
  *done = 0;
  if (ticket == IEKV_QUEUE_DONE) {
    *done = 1;
    return IEKV_OK;
  }
  std::lock_guard<std::mutex> lock(q->mu);
  if (q->broken) return queue_broken();
  if (ticket >= q->ticket_base + q->published)
    return set_error(IEKV_ERR_INVALID, "ticket %llu was not issued",
                     static_cast<unsigned long long>(ticket));
  if (ticket >= q->ticket_base) queue_retire(q);
  *done = ticket < q->ticket_base + q->retired ? 1 : 0;
  return IEKV_OK;
}

int iekv_queue_stop(iekv_queue* q) {
  if (!q) return set_error(IEKV_ERR_INVALID, "queue is null");
  std::lock_guard<std::mutex> lock(q->mu);
  DeviceGuard guard(q->src->device);
  if (!guard.ok()) return guard.fail();
  return queue_end(q);
}

int iekv_queue_destroy(iekv_queue* q) {
  if (!q) return IEKV_OK;
  int rc;
  {
    std::lock_guard<std::mutex> lock(q->mu);
    DeviceGuard guard(q->src->device);
    if (!guard.ok()) return guard.fail();
    rc = queue_end(q);
    // The kernel ends by its own limits even if the stop above timed out:
    // nothing it reads is freed before that.
    const hipError_t e = hipStreamSynchronize(q->stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      if (!rc) rc = set_error(IEKV_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    }
    (void)hipEventDestroy(q->ended);
    (void)hipStreamDestroy(q->stream);
    (void)hipFree(q->state);
    (void)hipHostFree(q->ring);
    (void)hipGetLastError();
  }
  delete q;
  return rc;
}

int iekv_queue_stats(const iekv_queue* q, uint64_t* descriptors, uint64_t* launches) {
  if (!q) return set_error(IEKV_ERR_INVALID, "queue is null");
  std::lock_guard<std::mutex> lock(const_cast<iekv_queue*>(q)->mu);
  if (descriptors) *descriptors = q->ticket_base + q->published;
  if (launches) *launches = q->launches;
  return IEKV_OK;
}

}  // extern "C"
