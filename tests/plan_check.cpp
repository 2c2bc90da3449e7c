// plan_check.cpp — CPU checks of the kv_move launch planning (kv_plan.h).
//
//  1. xcd_grouped is a bijection on [0, grid) for every grid up to 4,096 and
//     for large grids;
//  2. place_at visits every (unit, run, chunk) triple exactly once, for every
//     order, over many small shapes and the workloads' real shapes;
//  3. plan_move's shapes respect the dispatch limit, the chunk and tile-group
//     rules and the vector width, over a sweep of tiles, alignments, arrays,
//     block counts and settings;
//  4. simulating every launch and workgroup of small plans (each launch's
//     grid from launch_workgroups, as the host launches it, each workgroup
//     placed by place_in_grid, as the kernels place it) moves every vector of
//     every listed tile exactly once;
//  5. image_runs (the copies of a scattered restore) covers every image once,
//     in order, merges only images adjacent in memory within the allocation of
//     the run's first image, and merges every such pair: fixed layouts (one
//     allocation, neighbouring allocations, gaps, unknown memory, descending
//     addresses) and random ones;
//  6. image_views (device addresses of the direct host transfers) gives every
//     image its own allocation's address shift, looks each allocation up once
//     per stretch of images inside it, and refuses images in unmapped memory,
//     images running past their allocation's end and addresses whose end would
//     wrap, at the 70B-share workload's numbers (16,384 images of 2.5 MiB in one
//     64 GiB pinned allocation, or each in its own) and on random layouts
//     against a brute-force search;
//  7. images_per_launch and plan_slots cut every count of images into pieces
//     that stay within their byte limit and their staging slots (a simulated
//     pipeline writes only inside the staging buffer and covers every image
//     once); spans_cross agrees with a brute-force pairwise test.
// Built twice by the CPU test: optimised, and with AddressSanitizer and
// UndefinedBehaviorSanitizer (any report fails the run).
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

static const int32_t kOrders[] = {0, 1, 2, 3, 4, 5, 6, 7};

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
    // The grid the host launches, decoded the way the kernels decode it.
    const int grid = static_cast<int>(launch_workgroups(pl, runs));
    for (int i = 0; i < grid; ++i) {
      const Place p = place_in_grid(i, pl.units, runs, pl.parts, pl.order);
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

// Synthetic pinned allocations for image_views: [lo, hi) with a device shift.
struct Pinned {
  uint64_t lo, hi;
  int64_t shift;
  bool mapped;
};

struct HostMap {
  std::vector<Pinned> allocs;
  mutable int lookups = 0;
  HostSpan span(uint64_t p) const {
    ++lookups;
    HostSpan s;
    for (const Pinned& a : allocs)
      if (p >= a.lo && p < a.hi) {
        s.mapped = a.mapped;
        s.room = static_cast<int64_t>(a.hi - p);
        s.shift = a.shift;
      }
    return s;
  }
  // What a brute-force search says image [p, p + bytes) maps to (false: no view).
  bool expect(uint64_t p, int64_t bytes, uint64_t* view) const {
    for (const Pinned& a : allocs)
      if (a.mapped && p >= a.lo && p < a.hi && bytes <= static_cast<int64_t>(a.hi - p)) {
        *view = p + static_cast<uint64_t>(a.shift);
        return true;
      }
    return false;
  }
};

static bool views_of(const std::vector<uint64_t>& addresses, int64_t bytes, const HostMap& map,
                     std::vector<uint64_t>* out) {
  std::vector<const void*> images;
  for (uint64_t a : addresses) images.push_back(reinterpret_cast<const void*>(a));
  out->assign(addresses.size(), 0);
  return image_views(images.data(), static_cast<int32_t>(images.size()), bytes,
                     [&](uint64_t p) { return map.span(p); }, out->data());
}

static void check_image_views() {
  const int64_t img = 2621440;                     // a 70B-share block image, 2.5 MiB
  const int32_t n = 16384;                         // the 70B-share workload's blocks
  const uint64_t base = uint64_t(0x7f12) << 32;    // a host virtual address
  std::vector<uint64_t> addresses(n);
  for (int32_t i = 0; i < n; ++i) addresses[i] = base + static_cast<uint64_t>(i) * img;
  std::vector<uint64_t> views;

  // One pinned allocation holding every image, rounded up to 64 GiB.
  HostMap one{{{base, base + (uint64_t(1) << 36), 0, true}}};
  EXPECT(views_of(addresses, img, one, &views) && one.lookups == 1,
         "16,384 images in one allocation: one lookup (got %d)", one.lookups);
  EXPECT(views == addresses, "identity-mapped pinned memory keeps the host addresses");

  // The same images in an allocation of exactly their size: the last image ends
  // at the allocation's end and is accepted; one byte less refuses it.
  HostMap exact{{{base, base + static_cast<uint64_t>(n) * img, 4096, true}}};
  EXPECT(views_of(addresses, img, exact, &views) && views[n - 1] == addresses[n - 1] + 4096,
         "an allocation of exactly the images' size, with a device shift");
  HostMap short_by_one{{{base, base + static_cast<uint64_t>(n) * img - 1, 0, true}}};
  EXPECT(!views_of(addresses, img, short_by_one, &views),
         "the last image runs one byte past its allocation: no view");

  // Each image in its own exact-size allocation (the tier's one-block buffers),
  // allocations 4 KiB apart, each with its own shift; groups of 25 images as
  // one direct launch takes them (64 MiB / 2.5 MiB).
  HostMap own;
  std::vector<uint64_t> scattered;
  for (int32_t i = 0; i < 1024; ++i) {
    const uint64_t lo = base + static_cast<uint64_t>(i) * (img + 4096);
    own.allocs.push_back({lo, lo + img, int64_t(i) << 12, true});
    scattered.push_back(lo);
  }
  for (int32_t first = 0; first < 1024; first += 25) {
    const int32_t cnt = std::min<int32_t>(25, 1024 - first);
    std::vector<uint64_t> group(scattered.begin() + first, scattered.begin() + first + cnt);
    own.lookups = 0;
    bool ok = views_of(group, img, own, &views) && own.lookups == cnt;
    for (int32_t j = 0; ok && j < cnt; ++j)
      ok = views[j] == group[j] + (static_cast<uint64_t>(first + j) << 12);
    EXPECT(ok, "group at %d: each image takes its own allocation's shift", first);
  }

  // Unmapped memory anywhere in the list refuses the whole list.
  HostMap mixed{{{base, base + 8 * img, 0, true}, {base + 8 * img, base + 16 * img, 0, false}}};
  std::vector<uint64_t> sixteen(addresses.begin(), addresses.begin() + 16);
  EXPECT(!views_of(sixteen, img, mixed, &views), "an image in unmapped memory: no views");
  EXPECT(views_of(std::vector<uint64_t>(addresses.begin(), addresses.begin() + 8), img, mixed,
                  &views), "the mapped half alone has views");

  // Interior pointers and descending order: every image is looked up again once
  // it leaves the stretch [first looked-up address, allocation end).
  std::vector<uint64_t> down(addresses.rbegin(), addresses.rbegin() + 64);
  one.lookups = 0;
  EXPECT(views_of(down, img, one, &views) && views == down && one.lookups == 64,
         "descending images: one lookup each (%d)", one.lookups);

  // Degenerate sizes and addresses whose end would wrap around.
  EXPECT(!views_of({base}, 0, one, &views), "zero-byte images have no view");
  EXPECT(!views_of({UINT64_MAX - 100}, 4096, one, &views), "an image whose end wraps: no view");

  // Random layouts against the brute-force search.
  std::mt19937_64 rng(11);
  for (int trial = 0; trial < 4000; ++trial) {
    const int64_t size = int64_t(16) << (rng() % 10);
    HostMap map;
    uint64_t at = base;
    const int n_alloc = 1 + static_cast<int>(rng() % 5);
    for (int a = 0; a < n_alloc; ++a) {
      const uint64_t len = size * (1 + rng() % 5) + (rng() % 3 == 0 ? rng() % size : 0);
      map.allocs.push_back({at, at + len, static_cast<int64_t>(rng() % 3) << 20, rng() % 6 != 0});
      at += len + (rng() % 2 ? 0 : size);
    }
    std::vector<uint64_t> list;
    const int count = 1 + static_cast<int>(rng() % 12);
    for (int i = 0; i < count; ++i) {
      const Pinned& a = map.allocs[rng() % map.allocs.size()];
      list.push_back(a.lo + (rng() % ((a.hi - a.lo) / 16 + 1)) * 16);
    }
    bool want = true;
    std::vector<uint64_t> expected(list.size());
    for (size_t i = 0; i < list.size(); ++i) want = want && map.expect(list[i], size, &expected[i]);
    const bool got = views_of(list, size, map, &views);
    EXPECT(got == want, "random layout %d: views %d, brute force %d", trial, got, want);
    if (got && want) EXPECT(views == expected, "random layout %d: addresses differ", trial);
  }
}

static void check_pieces_and_slots() {
  const int64_t max_bytes = int64_t(64) << 20;
  // The direct launches of a restore: at most 128 images and 64 MiB each, one image
  // per launch when an image alone is larger.
  for (int64_t block : {int64_t(65536), int64_t(2) << 20, int64_t(2621440), int64_t(3) << 20,
                        int64_t(100) << 20})
    for (int32_t n : {1, 2, 24, 25, 26, 128, 129, 1024, 16384}) {
      const int32_t per = images_per_launch(n, block, max_bytes, 128);
      EXPECT(per >= 1 && per <= n && per <= 128, "per %d for %d images of %lld", per, n,
             static_cast<long long>(block));
      EXPECT(per * block <= max_bytes || per == 1, "%d images of %lld exceed a launch", per,
             static_cast<long long>(block));
      EXPECT(per == n || (per + 1) * block > max_bytes || per == 128,
             "%d images of %lld per launch: one more would fit", per,
             static_cast<long long>(block));
    }
  EXPECT(images_per_launch(16384, 2621440, max_bytes, 128) == 25,
         "2.5 MiB images: 25 per 64 MiB launch");

  // Staging slots: the pipeline's chunks stay inside the buffer and cover every
  // image once, alternating between the slots.
  int n_slots = 0;
  int64_t slot_blocks = 0;
  EXPECT(!plan_slots(2621440 - 1, 2621440, 10, &n_slots, &slot_blocks),
         "a buffer smaller than one image makes no progress: refused");
  EXPECT(!plan_slots(4096, 0, 10, &n_slots, &slot_blocks), "zero-byte images: refused");
  for (int64_t block : {int64_t(65536), int64_t(2621440), int64_t(3) << 20})
    for (int64_t staging : {block, 2 * block - 1, 2 * block, int64_t(512) << 20,
                            int64_t(256) << 20})
      for (int32_t n : {1, 2, 3, 101, 102, 103, 16384}) {
        if (!plan_slots(staging, block, n, &n_slots, &slot_blocks)) {
          EXPECT(false, "plan_slots refused %lld of staging for %lld-byte images",
                 static_cast<long long>(staging), static_cast<long long>(block));
          continue;
        }
        EXPECT(n_slots * slot_blocks * block <= staging, "slots overrun the staging buffer");
        int64_t covered = 0;
        for (int64_t first = 0, k = 0; first < n; first += slot_blocks, ++k) {
          const int64_t cnt = std::min<int64_t>(slot_blocks, n - first);
          const int64_t slot = (k % n_slots) * slot_blocks * block;
          EXPECT(slot + cnt * block <= staging, "chunk %lld writes past the staging buffer",
                 static_cast<long long>(k));
          covered += cnt;
        }
        EXPECT(covered == n, "chunks cover %lld of %d images", static_cast<long long>(covered),
               n);
      }
  EXPECT(plan_slots(int64_t(512) << 20, 2621440, 16384, &n_slots, &slot_blocks) &&
             n_slots == 2 && slot_blocks == 102,
         "512 MiB of staging: two slots of 102 images of 2.5 MiB");

  // spans_cross against a pairwise test.
  std::mt19937_64 rng(5);
  for (int trial = 0; trial < 3000; ++trial) {
    std::vector<Span> spans;
    const int count = 1 + static_cast<int>(rng() % 10);
    for (int i = 0; i < count; ++i) {
      const uint64_t lo = rng() % 64, len = rng() % 12;
      spans.push_back({lo, lo + len, static_cast<int>(rng() % 2)});
    }
    bool want = false;
    for (const Span& x : spans)
      for (const Span& y : spans)
        if (x.owner == 0 && y.owner == 1 && x.lo < y.hi && y.lo < x.hi && x.lo < x.hi &&
            y.lo < y.hi)
          want = true;
    EXPECT(spans_cross(spans) == want, "spans_cross trial %d", trial);
  }
}

// Which chunk each kind of launch takes (iekv_plan::launch_chunk), against the rule
// written out case by case: packs and offloads the staging chunk; pool-to-pool moves
// the pool-writing chunk; unpacks the pool-writing chunk for tiles at least that
// large or when it is 0 (whole tiles), else the staging chunk.
static void check_launch_chunk() {
  using iekv_plan::launch_chunk;
  for (int32_t staged : {0, 1024, 4096, 8192})
    for (int32_t pool : {0, 2048, 8192, 16384})
      for (int64_t tile : {16, 1024, 2048, 4096, 8192, 16384, 32768, 65536}) {
        EXPECT(launch_chunk(true, false, tile, staged, pool) == staged, "pack chunk");
        EXPECT(launch_chunk(false, false, tile, staged, pool) == staged, "host pack chunk");
        EXPECT(launch_chunk(true, true, tile, staged, pool) == pool, "direct chunk");
        const int32_t want = (pool == 0 || tile >= pool) ? pool : staged;
        EXPECT(launch_chunk(false, true, tile, staged, pool) == want,
               "unpack chunk: staged %d pool %d tile %lld", staged, pool, (long long)tile);
      }
  // The defaults on the benchmark workloads' tiles: 8 KiB and larger tiles are
  // unpacked in 8 KiB chunks, the tensor-parallel shares' 2 and 4 KiB tiles keep 4 KiB.
  EXPECT(launch_chunk(false, true, 32768, 4096, 8192) == 8192, "cfg3 unpack");
  EXPECT(launch_chunk(false, true, 8192, 4096, 8192) == 8192, "cfg1 / tp unpack");
  EXPECT(launch_chunk(false, true, 4096, 4096, 8192) == 4096, "cfg3 tp8 unpack");
  EXPECT(launch_chunk(false, true, 2048, 4096, 8192) == 4096, "cfg5 tp8 unpack");
}

// The request queue's claims (queue_claims): a descriptor's claims cover each
// (block, unit) pair exactly once, no claim is empty or spans two blocks, there
// are at most kQueueMaxClaims of them, a request no larger than the mover count
// is spread one unit per claim, and k reaches max_k for a large request unless
// the claim cap needs more. The claim ring then holds the claims of twice the
// descriptors that can be in flight, so the record of a claim still waiting is
// never rewritten: the claims between a record's two uses span at least
// 2 * slots descriptors, and a descriptor is published only after the one
// `slots` before it has finished.
static void check_queue_claims() {
  for (int64_t workers : {1, 7, 1024})
    for (int64_t max_k : {1, 4, 64})
      for (int64_t units : {1, 2, 3, 8, 10, 48, 64, 160, 65536})
        for (int64_t n_blocks : {1, 2, 5, 19, 64, 405, 1000, 1024}) {
          const QueueClaims c = queue_claims(n_blocks, units, workers, max_k);
          const int64_t n_units = n_blocks * units;
          EXPECT(c.k >= 1 && c.k <= units && c.per_block >= 1, "k %lld per block %lld",
                 (long long)c.k, (long long)c.per_block);
          EXPECT(c.n_claims == n_blocks * c.per_block && c.n_claims <= kQueueMaxClaims,
                 "%lld blocks x %lld units: %lld claims", (long long)n_blocks, (long long)units,
                 (long long)c.n_claims);
          EXPECT(c.per_block * c.k >= units && (c.per_block - 1) * c.k < units,
                 "units %lld: claims of %lld do not cover a block exactly", (long long)units,
                 (long long)c.k);
          if (n_units <= workers)
            EXPECT(c.k == 1, "n %lld <= workers %lld: k %lld", (long long)n_units,
                   (long long)workers, (long long)c.k);
          if (n_units / workers >= max_k && max_k <= units &&
              n_blocks * ((units + max_k - 1) / max_k) <= kQueueMaxClaims)
            EXPECT(c.k == max_k, "n %lld: k %lld, not max_k %lld", (long long)n_units,
                   (long long)c.k, (long long)max_k);
          if (n_units <= 200000) {   // brute force: every (block, unit) in exactly one claim
            std::vector<int> hit(static_cast<size_t>(n_units), 0);
            for (int64_t claim = 0; claim < c.n_claims; ++claim) {
              const int64_t b = claim / c.per_block, first = (claim % c.per_block) * c.k;
              const int64_t count = std::min(c.k, units - first);
              EXPECT(count >= 1, "claim %lld is empty", (long long)claim);
              for (int64_t u = first; u < first + count; ++u) ++hit[b * units + u];
            }
            for (int64_t u = 0; u < n_units; ++u)
              if (hit[u] != 1) {
                EXPECT(false, "unit %lld in %d claims", (long long)u, hit[u]);
                break;
              }
          }
        }
  EXPECT(queue_claims(0, 8, 1024, 4).n_claims == 0, "an empty descriptor has no claims");
  // Units of the queue's movers: a group of small tiles is moved by one wave, lane l
  // taking vector l % tile_vecs of a tile, so tile_vecs divides the wave; a group
  // stays within the chunk and the block's arrays.
  for (int64_t tile_vecs : {1, 2, 3, 4, 8, 16, 32, 48, 64, 128, 256, 2048})
    for (int vec : {1, 4, 16})
      for (int64_t chunk : {0, 1024, 8192})
        for (int32_t n_arrays : {1, 6, 64, 160}) {
          const int g = queue_tile_group(tile_vecs, vec, chunk, n_arrays);
          EXPECT(g >= 1 && g <= n_arrays, "group %d of %d arrays", g, n_arrays);
          if (g > 1)
            EXPECT(kQueueWave % tile_vecs == 0 && g * tile_vecs * vec <= chunk,
                   "group %d of %lld-vector tiles", g, (long long)tile_vecs);
          if (chunk > 0 && kQueueWave % tile_vecs == 0 && 2 * tile_vecs * vec <= chunk &&
              n_arrays > 1)
            EXPECT(g > 1, "small tiles (%lld vectors of %d B) left ungrouped", (long long)tile_vecs,
                   vec);
        }
  for (int64_t slots : {1, 16, 256})
    EXPECT(queue_claim_ring(slots) >= 2 * slots * kQueueMaxClaims, "claim ring too small");
}

int main() {
  check_queue_claims();
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
  check_image_views();
  check_pieces_and_slots();
  check_launch_chunk();

  if (failures) {
    std::printf("%d failures\n", failures);
    return 1;
  }
  std::printf("plan ok\n");
  return 0;
}
