/*
 * c_abi_handoff.c — the KV handoff driven from plain C through include/iekv.h,
 * with no Python or torch: two pools in one HIP allocation, the GPU-side check
 * of device id lists, a direct copy with device ids, the same with host ids
 * (kernel-argument ids), and a pack ->
 * unpack through a staging buffer. Every moved tile and every untouched tile
 * is checked byte for byte on the host. Then host offload / restore of the
 * moved blocks, through pinned memory (hipHostMalloc: the move kernel reads
 * and writes it directly) and through pageable memory (malloc: the staged
 * pipelines), each image checked on the host and restored into a cleared
 * pool. Exit status 0 and "c-abi handoff ok" on success.
 *
 * Built by __graft_entry__.build() with gcc into tests/c_abi_handoff (run by
 * tests/test_gpu_c_abi.py on a GPU).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "iekv.h"

#define ARRAYS 6      /* 2L for L = 3 */
#define TILE 4096     /* bytes per (array, block) tile */
#define BLOCKS 40     /* blocks per pool */
#define MOVED 12      /* blocks moved by each call */

#define CHECK_HIP(x)                                                              \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));              \
      return 2;                                                                   \
    }                                                                             \
  } while (0)
#define CHECK_IEKV(x)                                                             \
  do {                                                                            \
    int rc_ = (x);                                                                \
    if (rc_ != IEKV_OK) {                                                         \
      fprintf(stderr, "%s failed (%d): %s\n", #x, rc_, iekv_last_error());        \
      return 3;                                                                   \
    }                                                                             \
  } while (0)

static const size_t POOL = (size_t)ARRAYS * BLOCKS * TILE;

static unsigned char byte_at(int pool, int a, int b, int i) {
  return (unsigned char)(pool * 131 + a * 29 + b * 7 + i * 3 + (i >> 8));
}

/* dst tile (a, d) must equal src tile (a, s); other dst tiles keep their fill. */
static int check(const unsigned char* dst, const int* moved_to, const int* moved_from) {
  for (int a = 0; a < ARRAYS; ++a)
    for (int b = 0; b < BLOCKS; ++b) {
      const unsigned char* tile = dst + ((size_t)a * BLOCKS + b) * TILE;
      const int from = moved_from[b];
      for (int i = 0; i < TILE; ++i) {
        const unsigned char want = from >= 0 ? byte_at(0, a, from, i) : byte_at(1, a, b, i);
        if (tile[i] != want) {
          fprintf(stderr, "array %d block %d byte %d: %u != %u (moved %d)\n", a, b, i, tile[i],
                  want, moved_to[b]);
          return 1;
        }
      }
    }
  return 0;
}

int main(void) {
  unsigned char* host = (unsigned char*)malloc(2 * POOL);
  if (!host) return 4;
  for (int p = 0; p < 2; ++p)
    for (int a = 0; a < ARRAYS; ++a)
      for (int b = 0; b < BLOCKS; ++b)
        for (int i = 0; i < TILE; ++i)
          host[p * POOL + ((size_t)a * BLOCKS + b) * TILE + i] = byte_at(p, a, b, i);

  char* slab = NULL;
  CHECK_HIP(hipMalloc((void**)&slab, 2 * POOL));
  CHECK_HIP(hipMemcpy(slab, host, 2 * POOL, hipMemcpyHostToDevice));
  uint64_t src_arrays[ARRAYS], dst_arrays[ARRAYS];
  for (int a = 0; a < ARRAYS; ++a) {
    src_arrays[a] = (uint64_t)(uintptr_t)(slab + (size_t)a * BLOCKS * TILE);
    dst_arrays[a] = (uint64_t)(uintptr_t)(slab + POOL + (size_t)a * BLOCKS * TILE);
  }
  iekv_pool *src = NULL, *dst = NULL;
  CHECK_IEKV(iekv_pool_create(src_arrays, ARRAYS, TILE, BLOCKS, 0, &src));
  CHECK_IEKV(iekv_pool_create(dst_arrays, ARRAYS, TILE, BLOCKS, 0, &dst));

  /* Three disjoint batches of MOVED blocks: direct (device ids), direct (host
   * ids), pack -> unpack (device ids). */
  int s_ids[3][MOVED], d_ids[3][MOVED];
  int moved_from[BLOCKS], moved_to[BLOCKS];
  for (int b = 0; b < BLOCKS; ++b) moved_from[b] = moved_to[b] = -1;
  for (int k = 0; k < 3; ++k)
    for (int i = 0; i < MOVED; ++i) {
      s_ids[k][i] = (7 * (k * MOVED + i) + 3) % BLOCKS;
      d_ids[k][i] = (11 * (k * MOVED + i) + 5) % BLOCKS;
      moved_from[d_ids[k][i]] = s_ids[k][i];
      moved_to[d_ids[k][i]] = k;
    }
  int32_t* dev_ids = NULL;
  CHECK_HIP(hipMalloc((void**)&dev_ids, sizeof(int32_t) * 4 * MOVED));
  int32_t staged[4 * MOVED];
  for (int i = 0; i < MOVED; ++i) {
    staged[i] = s_ids[0][i];
    staged[MOVED + i] = d_ids[0][i];
    staged[2 * MOVED + i] = s_ids[2][i];
    staged[3 * MOVED + i] = d_ids[2][i];
  }
  CHECK_HIP(hipMemcpy(dev_ids, staged, sizeof(staged), hipMemcpyHostToDevice));
  void* staging = NULL;
  const int64_t staging_bytes = (int64_t)MOVED * ARRAYS * TILE;
  CHECK_HIP(hipMalloc(&staging, (size_t)staging_bytes));
  hipStream_t stream;
  CHECK_HIP(hipStreamCreate(&stream));

  /* The device id lists pass the GPU-side checks (status 0); a destination
   * list that names one block twice sets IEKV_IDS_DST_REPEATED. */
  int32_t* status = NULL;
  void* bitmap = NULL;
  CHECK_HIP(hipMalloc((void**)&status, sizeof(int32_t)));
  CHECK_HIP(hipMalloc(&bitmap, (size_t)IEKV_CHECK_WORKSPACE_BYTES(BLOCKS)));
  int32_t verdict = -1;
  CHECK_IEKV(iekv_check_ids(src, dev_ids, dst, dev_ids + MOVED, MOVED, bitmap,
                            IEKV_CHECK_WORKSPACE_BYTES(BLOCKS), status, stream));
  CHECK_HIP(hipMemcpyAsync(&verdict, status, sizeof(verdict), hipMemcpyDeviceToHost, stream));
  CHECK_HIP(hipStreamSynchronize(stream));
  if (verdict != 0) return 7;
  int32_t repeated[2] = {d_ids[0][0], d_ids[0][0]};
  int32_t* dev_repeated = NULL;
  CHECK_HIP(hipMalloc((void**)&dev_repeated, sizeof(repeated)));
  CHECK_HIP(hipMemcpy(dev_repeated, repeated, sizeof(repeated), hipMemcpyHostToDevice));
  CHECK_IEKV(iekv_check_ids(src, dev_ids, dst, dev_repeated, 2, bitmap,
                            IEKV_CHECK_WORKSPACE_BYTES(BLOCKS), status, stream));
  CHECK_HIP(hipMemcpyAsync(&verdict, status, sizeof(verdict), hipMemcpyDeviceToHost, stream));
  CHECK_HIP(hipStreamSynchronize(stream));
  if (verdict != IEKV_IDS_DST_REPEATED) return 7;
  CHECK_HIP(hipFree(dev_repeated));
  CHECK_HIP(hipFree(bitmap));
  CHECK_HIP(hipFree(status));

  CHECK_IEKV(iekv_copy_direct(src, dst, dev_ids, dev_ids + MOVED, MOVED, stream));
  CHECK_IEKV(iekv_copy_direct_ids(src, dst, s_ids[1], d_ids[1], MOVED, stream));
  CHECK_IEKV(iekv_pack(src, dev_ids + 2 * MOVED, MOVED, staging, staging_bytes, stream));
  CHECK_IEKV(iekv_unpack(dst, dev_ids + 3 * MOVED, MOVED, staging, staging_bytes, stream));
  CHECK_HIP(hipStreamSynchronize(stream));

  /* An out-of-range host id, and a destination given twice, are refused before
   * anything is enqueued. */
  int bad[1] = {BLOCKS};
  if (iekv_copy_direct_ids(src, dst, bad, d_ids[0], 1, stream) != IEKV_ERR_RANGE) return 5;
  int twice[2] = {d_ids[0][0], d_ids[0][0]};
  if (iekv_copy_direct_ids(src, dst, s_ids[0], twice, 2, stream) != IEKV_ERR_IDS) return 5;

  CHECK_HIP(hipMemcpy(host, slab, 2 * POOL, hipMemcpyDeviceToHost));
  if (check(host + POOL, moved_to, moved_from)) return 1;
  for (int a = 0; a < ARRAYS; ++a) /* the source pool is untouched */
    for (int b = 0; b < BLOCKS; ++b)
      for (int i = 0; i < TILE; ++i)
        if (host[((size_t)a * BLOCKS + b) * TILE + i] != byte_at(0, a, b, i)) return 6;

  /* Host offload of batch 0's source blocks, then restore onto batch 0's
   * destination blocks of a cleared destination pool: once through pinned
   * memory, once through pageable memory. */
  hipStream_t side;
  CHECK_HIP(hipStreamCreate(&side));
  const int64_t image_bytes = (int64_t)MOVED * ARRAYS * TILE;
  for (int pinned = 1; pinned >= 0; --pinned) {
    unsigned char* image = NULL;
    if (pinned) {
      CHECK_HIP(hipHostMalloc((void**)&image, (size_t)image_bytes, 0));
    } else {
      image = (unsigned char*)malloc((size_t)image_bytes);
      if (!image) return 4;
    }
    memset(image, 0, (size_t)image_bytes);
    CHECK_IEKV(iekv_offload(src, dev_ids, MOVED, image, image_bytes, staging, staging_bytes,
                            stream, side));
    CHECK_HIP(hipStreamSynchronize(stream));
    for (int k = 0; k < MOVED; ++k) /* image k = the 2L tiles of source block s_ids[0][k] */
      for (int a = 0; a < ARRAYS; ++a)
        for (int i = 0; i < TILE; ++i)
          if (image[((size_t)k * ARRAYS + a) * TILE + i] != byte_at(0, a, s_ids[0][k], i))
            return pinned ? 7 : 8;
    CHECK_HIP(hipMemset(slab + POOL, 0, POOL));
    CHECK_IEKV(iekv_restore(dst, dev_ids + MOVED, MOVED, image, image_bytes, staging,
                            staging_bytes, stream, side));
    CHECK_HIP(hipStreamSynchronize(side)); /* `side` is ordered after the last unpack */
    CHECK_HIP(hipMemcpy(host + POOL, slab + POOL, POOL, hipMemcpyDeviceToHost));
    for (int a = 0; a < ARRAYS; ++a)
      for (int b = 0; b < BLOCKS; ++b) {
        const unsigned char* tile = host + POOL + ((size_t)a * BLOCKS + b) * TILE;
        int from = -1;
        for (int k = 0; k < MOVED; ++k)
          if (d_ids[0][k] == b) from = s_ids[0][k];
        for (int i = 0; i < TILE; ++i)
          if (tile[i] != (from >= 0 ? byte_at(0, a, from, i) : 0)) return pinned ? 9 : 10;
      }
    if (pinned) {
      CHECK_HIP(hipHostFree(image));
    } else {
      free(image);
    }
  }
  CHECK_HIP(hipStreamDestroy(side));

  CHECK_IEKV(iekv_pool_destroy(src));
  CHECK_IEKV(iekv_pool_destroy(dst));
  CHECK_HIP(hipFree(staging));
  CHECK_HIP(hipFree(dev_ids));
  CHECK_HIP(hipFree(slab));
  CHECK_HIP(hipStreamDestroy(stream));
  free(host);
  printf("c-abi handoff ok: %d blocks x %d tiles of %d B in 4 calls, host round trips pinned "
         "and pageable\n", 3 * MOVED, ARRAYS, TILE);
  return 0;
}
