// plan_check.cpp — CPU checks of the kv_move launch planning (kv_plan.h).
//
//  1. xcd_grouped is a bijection on [0, grid) for every grid up to 4,096 and
//     for large grids;
//  2. place_at visits every (unit, run, chunk) triple exactly once, for every
//     order, over many small shapes and the workloads' real shapes;
//  3. plan_move's shapes respect the dispatch limit, the chunk and tile-group
//     rules and the vector width, over a sweep of tiles, alignments, arrays,
//     block counts and settings;
//  4. simulating every launch and workgroup of small plans moves every vector
//     of every listed tile exactly once;
//  5. image_runs (the copies of a scattered restore) covers every image once,
//     in order, merges only images adjacent in memory within the allocation of
//     the run's first image, and merges every such pair: fixed layouts (one
//     allocation, neighbouring allocations, gaps, unknown memory, descending
//     addresses) and random ones.
// Prints "plan ok" and exits 0, or names the first failure and exits 1.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "../inference-engine_amd/csrc/kv_plan.h"

using namespace iekv_plan;

static int failures = 0;
#define EXPECT(cond, ...)                        \
  do {                                           \
    if (!(cond)) {                               \
      if (failures++ < 10) {                     \
        std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
        std::printf(__VA_ARGS__);                \
        std::printf("\n");                       \
      }                                          \
    }                                            \
  } while (0)

static const int32_t kOrders[] = {0, 1, 2, 4, 5, 6};

static void check_xcd_grouped(int grid) {
  std::vector<char> seen(grid, 0);
  for (int i = 0; i < grid; ++i) {
    const int w = xcd_grouped(i, grid);
    EXPECT(w >= 0 && w < grid && !seen[w], "xcd_grouped(%d, %d) = %d", i, grid, w);
    if (w >= 0 && w < grid) seen[w] = 1;
  }
}

static void check_place(int32_t units, int32_t runs, int32_t parts, int32_t order) {
  const int grid = units * runs * parts;
  std::vector<char> seen(grid, 0);
  for (int i = 0; i < grid; ++i) {
    const Place pl = place_at(i, grid, units, runs, parts, order);
    const bool in = pl.a >= 0 && pl.a < units && pl.r >= 0 && pl.r < runs && pl.p >= 0 &&
                    pl.p < parts;
    EXPECT(in, "place_at out of range: units %d runs %d parts %d order %d", units, runs, parts,
           order);
    if (!in) return;
    const int key = (pl.a * runs + pl.r) * parts + pl.p;
    EXPECT(!seen[key], "place_at repeats a triple: units %d runs %d parts %d order %d", units,
           runs, parts, order);
    seen[key] = 1;
  }
}

static int pow2_divisor(int64_t x) {
  int a = 16;
  while (a > 1 && x % a) a >>= 1;
  return a;
}

static void check_plan(int32_t n_blocks, int64_t tile_bytes, int32_t n_arrays, int align,
                       bool single, const Settings& s) {
  MovePlan pl;
  const Status st = plan_move(n_blocks, tile_bytes, n_arrays, align, true, single, s, &pl);
  EXPECT(st == kPlanned, "plan refused: tile %lld arrays %d", (long long)tile_bytes, n_arrays);
  if (st != kPlanned) return;
  const int64_t tile_vecs = tile_bytes / pl.vec;
  EXPECT(pl.vec <= align && tile_bytes % pl.vec == 0 && (pl.vec & (pl.vec - 1)) == 0,
         "vector width %d for tile %lld align %d", pl.vec, (long long)tile_bytes, align);
  EXPECT(pl.run >= 1 && (!single || pl.run == 1) && (s.run <= 0 || single || pl.run == s.run),
         "run %d", pl.run);
  EXPECT(pl.parts >= 1 && (pl.parts & (pl.parts - 1)) == 0 && tile_vecs % pl.parts == 0,
         "parts %d of %lld vectors", pl.parts, (long long)tile_vecs);
  EXPECT(pl.run == 1 || pl.parts == 1, "runs of several blocks split tiles");
  if (pl.parts > 1)
    EXPECT(tile_vecs / pl.parts * pl.vec >= s.chunk_bytes, "chunk %lld below %lld",
           (long long)(tile_vecs / pl.parts * pl.vec), (long long)s.chunk_bytes);
  EXPECT(pl.group >= 1 && pl.group <= n_arrays, "group %d of %d arrays", pl.group, n_arrays);
  if (pl.group > 1)
    EXPECT(pl.run == 1 && pl.parts == 1 && kThreads % tile_vecs == 0 &&
               pl.group * tile_bytes <= s.chunk_bytes,
           "group %d: run %d parts %d tile %lld chunk %lld", pl.group, pl.run, pl.parts,
           (long long)tile_bytes, (long long)s.chunk_bytes);
  EXPECT(pl.units == (n_arrays + pl.group - 1) / pl.group, "units %d", pl.units);
  EXPECT(pl.total_runs == (int64_t(n_blocks) + pl.run - 1) / pl.run, "total runs");
  EXPECT(pl.runs_per_launch >= 1 && pl.runs_per_launch <= pl.total_runs &&
             pl.runs_per_launch * pl.units * pl.parts <= kMaxGrid,
         "runs per launch %lld (units %d parts %d)", (long long)pl.runs_per_launch, pl.units,
         pl.parts);
  const int64_t lane = (tile_vecs * pl.group / pl.parts + kThreads - 1) / kThreads;
  EXPECT(pl.lane_vecs == (lane < 16 ? lane : 16) && pl.lane_vecs >= 1, "lane vectors %d",
         pl.lane_vecs);
}

// Every workgroup of every launch of a plan, decoded the way kv_move decodes
// it: run r of the launch covers list entries [first + r*run, +run), unit a
// covers arrays [a*group, a*group+group), chunk p covers vectors
// [p*chunk, (p+1)*chunk) of each tile.
static void simulate(int32_t n_blocks, int64_t tile_bytes, int32_t n_arrays, int align,
                     const Settings& s, int32_t order) {
  MovePlan pl;
  Settings so = s;
  so.order = order;
  if (plan_move(n_blocks, tile_bytes, n_arrays, align, true, false, so, &pl) != kPlanned) return;
  const int64_t tile_vecs = tile_bytes / pl.vec;
  const int64_t chunk = tile_vecs / pl.parts;
  std::vector<int> hits(size_t(n_blocks) * n_arrays * tile_vecs, 0);
  for (int64_t r0 = 0; r0 < pl.total_runs; r0 += pl.runs_per_launch) {
    const int64_t first = r0 * pl.run;
    const int64_t cnt = std::min<int64_t>(pl.runs_per_launch * pl.run, n_blocks - first);
    const int32_t runs = int32_t((cnt + pl.run - 1) / pl.run);
    const int grid = runs * pl.units * pl.parts;
    for (int i = 0; i < grid; ++i) {
      const Place p = place_at(i, grid, pl.units, runs, pl.parts, pl.order);
      const int64_t e0 = first + int64_t(p.r) * pl.run;
      const int64_t e1 = std::min<int64_t>(e0 + pl.run, first + cnt);
      for (int64_t e = e0; e < e1; ++e)
        for (int a = p.a * pl.group; a < std::min(p.a * pl.group + pl.group, n_arrays); ++a)
          for (int64_t v = p.p * chunk; v < (p.p + 1) * chunk; ++v)
            ++hits[(size_t(e) * n_arrays + a) * tile_vecs + v];
    }
  }
  for (size_t k = 0; k < hits.size(); ++k) {
    EXPECT(hits[k] == 1, "vector %zu moved %d times (blocks %d tile %lld arrays %d order %d)",
           k, hits[k], n_blocks, (long long)tile_bytes, n_arrays, order);
    if (hits[k] != 1) return;
  }
}


// Synthetic allocations [lo, hi) for image_runs: room(address) is the distance
// to the end of the allocation holding it, 0 outside every allocation.
struct Allocations {
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  int64_t room(uint64_t address) const {
    for (const auto& r : ranges)
      if (address >= r.first && address < r.second) return static_cast<int64_t>(r.second - address);
    return 0;
  }
};

// The runs image_runs makes for `addresses`, as (first, count) pairs.
static std::vector<std::pair<int32_t, int32_t>> runs_of(const std::vector<uint64_t>& addresses,
                                                        int64_t image_bytes,
                                                        const Allocations& alloc) {
  std::vector<const void*> images;
  for (uint64_t a : addresses) images.push_back(reinterpret_cast<const void*>(a));
  std::vector<std::pair<int32_t, int32_t>> runs;
  image_runs(images.data(), static_cast<int32_t>(images.size()), image_bytes,
             [&](uint64_t a) { return alloc.room(a); },
             [&](int32_t first, int32_t count) { runs.emplace_back(first, count); });
  return runs;
}

// The properties every split must have: runs cover [0, n) in order; inside a
// run the images follow each other and stay within the allocation of its
// first image; and a run ends only where the next image is not adjacent or
// would cross that allocation's end (the split is as coarse as allowed).
static void check_runs(const std::vector<uint64_t>& addresses, int64_t image_bytes,
                       const Allocations& alloc, const char* what) {
  const auto runs = runs_of(addresses, image_bytes, alloc);
  int32_t next = 0;
  for (const auto& run : runs) {
    const int32_t first = run.first, count = run.second;
    EXPECT(first == next && count >= 1, "%s: run (%d, %d) does not continue at %d", what, first,
           count, next);
    const uint64_t start = addresses[first];
    const int64_t room = alloc.room(start);
    if (count > 1)
      EXPECT(count * image_bytes <= room, "%s: run at %d crosses its allocation's end", what,
             first);
    for (int32_t j = 1; j < count; ++j)
      EXPECT(addresses[first + j] == start + j * image_bytes, "%s: run at %d merges image %d, "
             "which is not adjacent", what, first, first + j);
    const int32_t end = first + count;
    if (end < static_cast<int32_t>(addresses.size()))
      EXPECT(addresses[end] != start + count * image_bytes || (count + 1) * image_bytes > room,
             "%s: run at %d stops before image %d, which it could take", what, first, end);
    next = end;
  }
  EXPECT(next == static_cast<int32_t>(addresses.size()), "%s: runs end at %d of %zu", what, next,
         addresses.size());
}

static void check_image_runs() {
  const int64_t img = 2 << 20;   // a Llama-3-8B-shape block image
  const uint64_t base = uint64_t(1) << 40;
  std::vector<uint64_t> eight;
  for (int i = 0; i < 8; ++i) eight.push_back(base + i * img);

  Allocations one{{{base, base + 8 * img}}};
  EXPECT(runs_of(eight, img, one) == (std::vector<std::pair<int32_t, int32_t>>{{0, 8}}),
         "8 adjacent images in one allocation are one copy");
  check_runs(eight, img, one, "one allocation");

  Allocations separate;
  for (int i = 0; i < 8; ++i) separate.ranges.push_back({base + i * img, base + (i + 1) * img});
  EXPECT(runs_of(eight, img, separate).size() == 8,
         "8 images in 8 neighbouring allocations are 8 copies");
  check_runs(eight, img, separate, "neighbouring allocations");

  Allocations split{{{base, base + 3 * img}, {base + 3 * img, base + 8 * img}}};
  EXPECT(runs_of(eight, img, split) == (std::vector<std::pair<int32_t, int32_t>>{{0, 3}, {3, 5}}),
         "adjacent images across an allocation boundary split there");
  check_runs(eight, img, split, "allocation boundary");

  Allocations unknown;
  EXPECT(runs_of(eight, img, unknown).size() == 8, "images in unknown memory are copied alone");

  std::vector<uint64_t> gapped = {base, base + img, base + 3 * img, base + 4 * img,
                                  base + 5 * img + 64};
  Allocations big{{{base, base + 16 * img}}};
  EXPECT(runs_of(gapped, img, big) ==
             (std::vector<std::pair<int32_t, int32_t>>{{0, 2}, {2, 2}, {4, 1}}),
         "a gap ends a run");
  check_runs(gapped, img, big, "gaps");

  std::vector<uint64_t> descending(eight.rbegin(), eight.rend());
  EXPECT(runs_of(descending, img, one).size() == 8, "descending images are copied alone");

  // An allocation that ends inside the second image: the first is copied alone.
  Allocations short_alloc{{{base, base + img + img / 2}}};
  EXPECT(runs_of({base, base + img}, img, short_alloc).size() == 2,
         "a run never extends past its allocation's end");

  // Random layouts: images drawn from a few allocations, mostly in ascending
  // runs with occasional jumps, gaps and repeats of neighbouring buffers.
  std::mt19937_64 rng(7);
  for (int trial = 0; trial < 3000; ++trial) {
    const int64_t size = int64_t(64) << (rng() % 6);
    Allocations alloc;
    uint64_t at = base;
    const int n_alloc = 1 + static_cast<int>(rng() % 6);
    for (int a = 0; a < n_alloc; ++a) {
      const uint64_t len = size * (1 + rng() % 6) + (rng() % 3 == 0 ? size / 2 : 0);
      alloc.ranges.push_back({at, at + len});
      at += len + (rng() % 2 ? 0 : size);   // neighbouring or separated allocations
    }
    std::vector<uint64_t> addresses;
    const int n = 1 + static_cast<int>(rng() % 24);
    uint64_t cursor = alloc.ranges[0].first;
    for (int i = 0; i < n; ++i) {
      const int pick = static_cast<int>(rng() % 8);
      if (pick == 0) cursor = alloc.ranges[rng() % alloc.ranges.size()].first;
      else if (pick == 1) cursor += size / 2;
      else if (pick == 2 && cursor > base + size) cursor -= size;
      addresses.push_back(cursor);
      cursor += size;
    }
    check_runs(addresses, size, alloc, "random layout");
  }
}

int main() {
  for (int grid = 1; grid <= 4096; ++grid) check_xcd_grouped(grid);
  for (int grid : {98816, 1048575, 4194304, 16777215}) check_xcd_grouped(grid);

  for (int32_t order : kOrders)
    for (int32_t units = 1; units <= 12; ++units)
      for (int32_t runs = 1; runs <= 12; ++runs)
        for (int32_t parts : {1, 2, 4, 8}) check_place(units, runs, parts, order);
  for (int32_t order : kOrders) {
    check_place(64, 193, 8, order);    // a mean Llama-3-8B-shape request, 4 KiB chunks
    check_place(80, 1024, 1, order);   // the 70B share at tp=8: 160 arrays in pairs
    check_place(160, 1024, 4, order);  // the 70B share, 16 KiB tiles in 4 KiB chunks
    check_place(7, 1, 3, order);       // a grid smaller than the 8 XCDs
  }

  const int64_t tiles[] = {1, 2, 3, 16, 30, 45, 48, 64, 192, 1024, 2048, 3072, 4096,
                           8192, 16384, 32768, 49152, 65536, 1 << 20};
  const int32_t arrays[] = {1, 2, 6, 10, 64, 160};
  const int32_t blocks[] = {1, 17, 193, 1024, 70000, 9000000};
  const int runs_setting[] = {0, 1, 3, 64};
  const int64_t chunks[] = {0, 64, 1024, 4096, 8192, 1 << 20};
  for (int64_t tile : tiles)
    for (int32_t n_arrays : arrays)
      for (int32_t n_blocks : blocks)
        for (int run : runs_setting)
          for (int64_t chunk : chunks)
            for (bool single : {false, true}) {
              Settings s;
              s.run = run;
              s.chunk_bytes = chunk;
              const int align = pow2_divisor(tile);
              check_plan(n_blocks, tile, n_arrays, align, single, s);
              if (align > 1) check_plan(n_blocks, tile, n_arrays, align / 2, single, s);
            }
  {  // the limits
    MovePlan pl;
    Settings s;
    s.chunk_bytes = 4096;
    EXPECT(plan_move(1, int64_t(1) << 32, 2, 1, true, false, s, &pl) == kTileTooLarge,
           "a 4 GiB tile of bytes is too large");
    EXPECT(plan_move(1, 16, int32_t(kMaxGrid) + 1, 16, true, false, s, &pl) == kTooManyArrays,
           "more arrays than one dispatch holds");
    EXPECT(plan_move(70000, 4096, 4, 16, true, false, [] {
             Settings c; c.chunk_bytes = 64; return c; }(), &pl) == kPlanned &&
               pl.parts == 32 && pl.runs_per_launch == 70000,
           "a split over the dispatch limit is halved to 32 chunks in one launch");
  }

  for (int32_t order : kOrders)
    for (int64_t tile : {16, 48, 64, 192, 2048, 4096, 8192, 32768})
      for (int32_t n_arrays : {1, 2, 6, 10})
        for (int64_t chunk : {0, 1024, 4096, 8192})
          for (int run : {0, 3}) {
            Settings s;
            s.run = run;
            s.chunk_bytes = chunk;
            simulate(13, tile, n_arrays, pow2_divisor(tile), s, order);
          }

  check_image_runs();

  if (failures) {
    std::printf("%d failures\n", failures);
    return 1;
  }
  std::printf("plan ok\n");
  return 0;
}
