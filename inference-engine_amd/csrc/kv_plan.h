// kv_plan.h — launch planning of the kv_move kernels in kv_handoff.hip: which
// workgroup moves which (array, list entry, chunk of a tile), and how one move
// is cut into launches. Plain functions for the host and for device code, so
// the CPU tests can check them over many shapes without a GPU.
#ifndef IEKV_KV_PLAN_H_
#define IEKV_KV_PLAN_H_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

namespace iekv_plan {

constexpr int kThreads = 256;   // four wave64 per workgroup
constexpr int kXcds = 8;        // MI355X: the dispatcher deals workgroups to 8 XCDs in turn
constexpr int kXcdGrouped = 4;  // order flag: give each XCD a contiguous share of the work
enum Order : int32_t { kArrayMajor = 0, kBlockMajor = 1, kDiagonal = 2, kScattered = 3 };
// Multiplier of the scattered order: a prime above every unit-run count a
// launch can hold (at most kMaxGrid), so u -> u * kScatterMul mod count is a
// bijection; 2654435761 is the prime nearest 2^32 / golden ratio, which spreads
// consecutive positions far apart.
constexpr int64_t kScatterMul = 2654435761LL;

// A dispatch holds at most 2^32 - 1 work-items, so one launch takes at most
// this many workgroups; larger moves are split over several launches.
constexpr int64_t kMaxGrid = static_cast<int64_t>(UINT32_MAX) / kThreads;

// One workgroup per (unit a, run of list entries, chunk p of each tile). A unit
// is one array, or with tile groups `group` consecutive arrays. A tile of
// tile_vecs vectors splits into `parts` chunks of tile_vecs / parts vectors;
// the workgroup moves chunk p of every tile in its run. The order in which
// workgroups take (unit, run) pairs decides which tiles are in flight
// together. With u the pair's position in that order:
//   kArrayMajor  u = run * n_units + a: the 2L tiles of one block; their
//                addresses differ by multiples of the array stride;
//   kBlockMajor  u = a * runs + run: random blocks of one array;
//   kDiagonal    as array-major, but unit a takes run (run + a) mod runs, so
//                the tiles in flight span 2L arrays AND 2L different blocks;
//   kScattered   array-major position v = u * kScatterMul mod (units * runs):
//                the (array, block) pairs in flight are spread over the whole
//                move, so its reads and writes hit unrelated addresses.
// The chunks of one tile are consecutive: position w = u * parts + p.
// Plain orders take w = the workgroup index. The dispatcher deals consecutive
// workgroups to the kXcds XCDs in turn, so with the kXcdGrouped flag set,
// workgroup i (on XCD i mod kXcds) takes position w = start(XCD) + i / kXcds
// instead: each XCD walks one contiguous share of the order (with
// kBlockMajor, its own eighth of the arrays). Every order covers each
// (unit, run, chunk) triple exactly once.

// Position of workgroup `i` of `grid` when each XCD takes a contiguous share:
// XCD x receives workgroups x, x + kXcds, ...; the first `grid % kXcds` XCDs
// receive one more than the rest. A bijection on [0, grid).
__host__ __device__ inline int xcd_grouped(int i, int grid) {
  const int q = grid / kXcds, rem = grid % kXcds;
  const int x = i % kXcds;
  return x * q + (x < rem ? x : rem) + i / kXcds;
}

struct Place {
  int a, r, p;  // unit, run, chunk
};

// The (unit, run, chunk) of workgroup `i` of a grid of n_units * runs * parts.
__host__ __device__ inline Place place_at(int i, int grid, int32_t n_units, int32_t runs,
                                          int32_t parts, int32_t order) {
  const int w = (order & kXcdGrouped) ? xcd_grouped(i, grid) : i;
  const int base_order = order & ~kXcdGrouped;
  Place pl;
  pl.p = w % parts;
  const int u = w / parts;
  if (base_order == kBlockMajor) {
    pl.a = u / runs;
    pl.r = u % runs;
  } else if (base_order == kScattered) {
    const int64_t count = static_cast<int64_t>(n_units) * runs;
    const int64_t v = static_cast<int64_t>(u) * kScatterMul % count;
    pl.a = static_cast<int>(v % n_units);
    pl.r = static_cast<int>(v / n_units);
  } else {
    pl.a = u % n_units;
    pl.r = u / n_units;
    if (base_order == kDiagonal)
      pl.r = static_cast<int>((static_cast<int64_t>(pl.r) + pl.a) % runs);
  }
  return pl;
}

// The same for a launch of exactly n_units * runs * parts workgroups, as every
// move launch is: the grid size follows from the plan, so a kernel need not
// read it from the dispatch. (A kernel that reads gridDim makes the runtime
// append its 256-byte block of hidden arguments to every launch's argument
// segment, and copying arguments is most of a small launch's host cost.)
__host__ __device__ inline Place place_in_grid(int i, int32_t n_units, int32_t runs,
                                               int32_t parts, int32_t order) {
  return place_at(i, n_units * runs * parts, n_units, runs, parts, order);
}

// Chunk size of a launch: a pool-to-pool move takes the pool-writing chunk; an
// unpack (staging to pool) takes it when its tiles are at least that large (they
// are then split into pool-writing chunks), else the staging chunk, which groups
// small tiles as the pack does; a launch that writes a staging image takes the
// staging chunk. 0 means whole tiles.
inline int32_t launch_chunk(bool pool_reading, bool pool_writing, int64_t tile_bytes,
                            int32_t staging_chunk, int32_t pool_chunk) {
  if (!pool_writing) return staging_chunk;
  return pool_reading || pool_chunk == 0 || tile_bytes >= pool_chunk ? pool_chunk
                                                                      : staging_chunk;
}

// Chunks per tile for a requested chunk size: the largest power of two that
// divides the tile's vector count and leaves chunks of at least chunk_bytes
// (1 when chunk_bytes is 0 or the tile is no larger than the chunk).
inline int chunk_parts(int64_t tile_vecs, int vec_bytes, int64_t chunk_bytes) {
  if (chunk_bytes <= 0) return 1;
  int parts = 1;
  while (tile_vecs % (2 * parts) == 0 && (tile_vecs / (2 * parts)) * vec_bytes >= chunk_bytes)
    parts *= 2;
  return parts;
}

// Tiles per workgroup for tiles smaller than the chunk size: chunk_bytes /
// tile bytes tiles of one block in consecutive arrays (at most n_arrays), when
// a tile's vector count divides the workgroup's lanes; 1 otherwise. Measured
// on MI355X on one rank's share of the 70B-share workload at tp=8 (2 KiB
// tiles, 160 arrays): two tiles per workgroup (4 KiB chunks) raised the
// per-request direct copy from 4.17 to 5.76 TB/s and pack -> unpack from 4.34
// to 6.15 TB/s; groups of 8 and 16 KiB were no faster.
inline int tile_group(int64_t tile_vecs, int vec_bytes, int64_t chunk_bytes, int32_t n_arrays) {
  if (chunk_bytes <= 0 || tile_vecs * vec_bytes >= chunk_bytes || kThreads % tile_vecs) return 1;
  const int64_t group = chunk_bytes / (tile_vecs * vec_bytes);
  return static_cast<int>(group < n_arrays ? group : n_arrays);
}

// The launch-shape settings a plan reads (iekv_set_launch).
struct Settings {
  int run = 0;               // blocks per workgroup run; 0 = automatic (one)
  int64_t chunk_bytes = 0;   // bytes per workgroup (see chunk_parts, tile_group)
  int32_t order = 0;         // order of launches that write a pool
  int32_t pack_order = 0;    // order of launches that write a staging buffer
};

// Launch shape of one move: blocks per run, chunks per tile, tiles per
// workgroup (group; then `units` array groups), vector width, vectors per
// lane per workgroup, workgroup order, and how many runs one launch takes.
struct MovePlan {
  int run = 1;
  int parts = 1;
  int group = 1;
  int32_t units = 0;
  int vec = 16;
  int lane_vecs = 1;
  int32_t tile_vecs = 0;
  int32_t order = 0;
  int64_t total_runs = 0;
  int64_t runs_per_launch = 0;
};

enum Status { kPlanned = 0, kTileTooLarge = 1, kTooManyArrays = 2 };

// The shape of a move of n_blocks list entries of n_arrays tiles of
// tile_bytes each, whose addresses are all multiples of `align` (a power of
// two <= 16). `single_blocks` forces one block per workgroup (the kernel with
// ids in its arguments). Runs of several tiles keep whole tiles per
// workgroup; single-tile workgroups split each tile into chunks, halving the
// split while a launch would not fit the dispatch limit, or group small
// tiles. A launch takes runs_per_launch runs: the grid of one launch is at
// most runs_per_launch * units * parts <= kMaxGrid workgroups.
inline Status plan_move(int32_t n_blocks, int64_t tile_bytes, int32_t n_arrays, int align,
                        bool pool_writing, bool single_blocks, const Settings& s,
                        MovePlan* pl) {
  // One block per workgroup unless set otherwise: the fastest shape measured
  // for every tile size the workloads use (more, smaller workgroups balance
  // the tail of each launch better than runs of several tiles do).
  pl->run = single_blocks ? 1 : (s.run > 0 ? s.run : 1);
  pl->vec = 16;
  for (int a = 16; a > align; a >>= 1) pl->vec = a >> 1;
  const int64_t tile_vecs = tile_bytes / pl->vec;
  if (tile_vecs > INT32_MAX) return kTileTooLarge;
  pl->parts = pl->run == 1 ? chunk_parts(tile_vecs, pl->vec, s.chunk_bytes) : 1;
  while (pl->parts > 1 && static_cast<int64_t>(n_arrays) * pl->parts > kMaxGrid) pl->parts /= 2;
  if (static_cast<int64_t>(n_arrays) * pl->parts > kMaxGrid) return kTooManyArrays;
  pl->total_runs = (static_cast<int64_t>(n_blocks) + pl->run - 1) / pl->run;
  while (pl->parts > 1 && pl->total_runs * n_arrays * pl->parts > kMaxGrid) pl->parts /= 2;
  pl->group = pl->run == 1 && pl->parts == 1
                  ? tile_group(tile_vecs, pl->vec, s.chunk_bytes, n_arrays) : 1;
  pl->units = (n_arrays + pl->group - 1) / pl->group;
  const int64_t lane_vecs = (tile_vecs * pl->group / pl->parts + kThreads - 1) / kThreads;
  pl->lane_vecs = static_cast<int>(lane_vecs < 16 ? lane_vecs : 16);
  pl->tile_vecs = static_cast<int32_t>(tile_vecs);
  pl->order = pool_writing ? s.order : s.pack_order;
  const int64_t fit = kMaxGrid / (static_cast<int64_t>(pl->units) * pl->parts);
  pl->runs_per_launch = pl->total_runs < fit ? pl->total_runs : fit;
  return kPlanned;
}

// Workgroups of one launch of a plan that covers `runs` runs (at most
// runs_per_launch): every launch of the move kernels has exactly this many,
// and the kernels rely on it (place_in_grid derives the grid size from the
// same three factors instead of reading it from the dispatch).
inline uint32_t launch_workgroups(const MovePlan& pl, int64_t runs) {
  return static_cast<uint32_t>(runs * pl.units * pl.parts);
}

// Copies of a scattered restore (iekv_restore_blocks): list entry i's host
// image of image_bytes bytes starts at address images[i]. Consecutive entries
// whose images follow each other in memory are copied with one transfer, but
// a run never extends past the end of the allocation that holds its first
// image: separately allocated buffers can be neighbours in the address space,
// and one copy must not read past the end of its source allocation.
// room(address) gives the bytes from `address` to the end of the allocation
// holding it (0 when unknown, which leaves each image on its own). emit(first,
// count) is called once per run, in list order; the runs cover [0, n).
template <typename Room, typename Emit>
inline void image_runs(const void* const* images, int32_t n, int64_t image_bytes, Room room,
                       Emit emit) {
  for (int32_t i = 0; i < n;) {
    const uint64_t start = reinterpret_cast<uint64_t>(images[i]);
    const int64_t space = room(start);
    int32_t len = 1;
    while (i + len < n &&
           reinterpret_cast<uint64_t>(images[i + len]) ==
               start + static_cast<uint64_t>(len) * static_cast<uint64_t>(image_bytes) &&
           static_cast<int64_t>(len + 1) * image_bytes <= space)
      ++len;
    emit(i, len);
    i += len;
  }
}

// What the runtime reports for the host allocation holding one address: whether
// it is pinned memory mapped for the device, the distance from the address to
// the allocation's end, and device address minus host address (the same for
// every byte of the allocation).
struct HostSpan {
  bool mapped = false;
  int64_t room = 0;
  int64_t shift = 0;
};

// Device addresses of n host images of `bytes` each (the direct host
// transfers): out[i] = images[i] + shift of the allocation holding it. One
// lookup per allocation: an image that lies inside [first looked-up address,
// end of its allocation) reuses that lookup. False when an image is not in
// mapped pinned memory or runs past its allocation's end; out is then
// partly written. lookup(address) returns the HostSpan of that address.
template <typename Lookup>
inline bool image_views(const void* const* images, int32_t n, int64_t bytes, Lookup lookup,
                        uint64_t* out) {
  if (bytes <= 0) return false;
  uint64_t lo = 0, hi = 0;
  int64_t shift = 0;
  bool have = false;
  for (int32_t i = 0; i < n; ++i) {
    const uint64_t p = reinterpret_cast<uint64_t>(images[i]);
    if (p > UINT64_MAX - static_cast<uint64_t>(bytes)) return false;
    if (!(have && p >= lo && p + static_cast<uint64_t>(bytes) <= hi)) {
      const HostSpan span = lookup(p);
      if (!span.mapped || span.room < bytes) return false;
      lo = p;
      hi = p + static_cast<uint64_t>(span.room);
      shift = span.shift;
      have = true;
    }
    out[i] = p + static_cast<uint64_t>(shift);
  }
  return true;
}

// Block images per launch of a direct host transfer: at most max_images, and at
// most max_bytes of images unless a single image is larger (then one per launch).
inline int32_t images_per_launch(int32_t n_blocks, int64_t block_bytes, int64_t max_bytes,
                                 int32_t max_images) {
  int64_t per = block_bytes > 0 ? max_bytes / block_bytes : 1;
  if (per > max_images) per = max_images;
  if (per > n_blocks) per = n_blocks;
  return static_cast<int32_t>(per < 1 ? 1 : per);
}

// Staging slots of a host pipeline: two when the buffer holds two block images
// or more, else one, each of slot_blocks images (at most n_blocks). False when
// the buffer cannot hold one image: the pipeline would make no progress.
inline bool plan_slots(int64_t staging_bytes, int64_t block_bytes, int32_t n_blocks,
                       int* n_slots, int64_t* slot_blocks) {
  const int64_t fit = block_bytes > 0 ? staging_bytes / block_bytes : 0;
  *n_slots = fit >= 2 ? 2 : 1;
  *slot_blocks = fit / *n_slots < n_blocks ? fit / *n_slots : n_blocks;
  return *slot_blocks >= 1;
}

// A byte range [lo, hi) of owner 0 or 1 (one pool's array, say).
struct Span {
  uint64_t lo, hi;
  int owner;
};

// Whether a span of owner 0 shares a byte with a span of owner 1. Sorted by
// start, a span meets an earlier span of the other owner exactly when that
// owner's furthest end so far lies past its start.
inline bool spans_cross(std::vector<Span> spans) {
  std::sort(spans.begin(), spans.end(),
            [](const Span& x, const Span& y) { return x.lo < y.lo; });
  uint64_t reach[2] = {0, 0};
  for (const Span& s : spans) {
    if (s.hi <= s.lo) continue;
    if (reach[1 - s.owner] > s.lo) return true;
    if (s.hi > reach[s.owner]) reach[s.owner] = s.hi;
  }
  return false;
}

// Request queue (iekv_queue_*). A descriptor's n_blocks blocks have `units`
// units each (a unit is one tile, or one group of small tiles); it is served in
// claims of at most k consecutive units of one block, so the claim's record can
// carry that block's id pair. Movers take claims from one cursor that runs over
// every descriptor of a session, and a ring of kQueueClaimRing records maps a
// claim to its work. A descriptor has at most kQueueMaxClaims claims, so the
// claims of `slots` descriptors in flight fill at most half the ring: a record
// is rewritten only after the descriptor of the claim it held has finished.
constexpr int64_t kQueueMaxClaims = 4096;

constexpr int64_t queue_claim_ring(int64_t slots) { return 2 * slots * kQueueMaxClaims; }

// Lanes that move one unit: each wave of the queue's kernel is a mover.
constexpr int kQueueWave = 64;

// Tiles per unit of the queue's movers: small tiles whose vector count divides
// the wave are grouped, chunk_bytes / tile bytes tiles of one block in
// consecutive arrays (at most n_arrays); any other tile is a unit of its own.
inline int queue_tile_group(int64_t tile_vecs, int vec_bytes, int64_t chunk_bytes,
                            int32_t n_arrays) {
  if (chunk_bytes <= 0 || tile_vecs * vec_bytes >= chunk_bytes || kQueueWave % tile_vecs)
    return 1;
  const int64_t group = chunk_bytes / (tile_vecs * vec_bytes);
  return static_cast<int>(group > n_arrays ? n_arrays : group);
}

struct QueueClaims {
  int64_t k = 1;          // units per claim (the last claim of a block may hold fewer)
  int64_t per_block = 0;  // claims per block: ceil(units / k)
  int64_t n_claims = 0;   // n_blocks * per_block
};

// Claims of a descriptor: spread over all `workers` (one unit per claim for a
// request no larger than the mover count), at most max_k units and at most one
// block per claim, and never more than kQueueMaxClaims claims (n_blocks is at
// most kQueueMaxClaims). Claim c is block c / per_block, units
// (c % per_block) * k onward.
inline QueueClaims queue_claims(int64_t n_blocks, int64_t units, int64_t workers,
                                int64_t max_k) {
  QueueClaims c;
  if (n_blocks <= 0 || units <= 0) return c;
  const int64_t n_units = n_blocks * units;
  int64_t k = workers > 0 ? n_units / workers : n_units;
  if (k > max_k) k = max_k;
  if (k > units) k = units;
  if (k < 1) k = 1;
  const int64_t most = kQueueMaxClaims / n_blocks > 0 ? kQueueMaxClaims / n_blocks : 1;
  const int64_t least_k = (units + most - 1) / most;
  if (k < least_k) k = least_k;
  c.k = k;
  c.per_block = (units + k - 1) / k;
  c.n_claims = n_blocks * c.per_block;
  return c;
}

}  // namespace iekv_plan

#endif  // IEKV_KV_PLAN_H_
