/*
 * iekv.h — C-ABI of the MI355X (gfx950) KV-cache handoff library, libiekv.so.
 *
 * The reference engine (kuluruvineeth/inference-engine) moves KV bytes only in
 * Python: LayeredSlotCopier.read_block / write_block (ie/engine/copier.py:18-31)
 * behind the SlotCopier protocol (ie/core/offload.py:8-11), driven per block by
 * PrefillWorker.prefill (ie/serve/disaggregated.py:50), DecodeWorker.admit
 * (ie/serve/disaggregated.py:81-82), BlockManager._forget (offload,
 * ie/core/block_manager.py:82) and BlockManager.allocate (restore,
 * ie/core/block_manager.py:159-162). Each entry point below replaces one of
 * those loops with one batched launch; the comment on each names the lines.
 *
 * Data model.
 *   A pool is the paged KV cache of one engine: 2L arrays (K of layers 0..L-1,
 *   then V of layers 0..L-1), each [num_blocks * block_size, H, D] contiguous,
 *   exactly the reference's per-layer caches (ie/kernels/reference.py:39-42,
 *   ie/kernels/torch_backend.py:6-10). Block b of array a is the contiguous
 *   tile [b*T, (b+1)*T) bytes of that array, T = block_size*H*D*elem_bytes
 *   (the slice copier.py:14-16 takes).
 *   A staging buffer is block-major [n_blocks][2L][T] bytes: entry i holds the
 *   2L tiles of the i-th listed block, K layers first, then V layers — the
 *   byte image of the reference payload ([K_0..K_{L-1}], [V_0..V_{L-1}])
 *   (copier.py:21-22).
 *   Block ids are int32 in DEVICE memory, except for the *_ids entry points,
 *   which take ids in HOST memory and check them before launching. Callers validate device ids against the pool size
 *   before a call; kernels skip a tile whose id is out of range so a bad id
 *   can never address memory outside the pool. The tiles of one call are
 *   moved concurrently: destination ids must be distinct, and a direct copy
 *   within one pool must not use a block as both source and destination
 *   (the calls taking device ids check neither; iekv_check_ids checks a
 *   device list on the GPU, and the host-id calls check their own).
 *   All copies are raw bytes: fp32/fp16/bf16/fp8/int8 caches move bit-exactly.
 *
 * Errors. Every function returns IEKV_OK (0) or a negative IEKV_ERR_* code,
 * and iekv_last_error() describes the last failure on the calling thread.
 * Argument errors are detected before anything is enqueued.
 *
 * Streams. Work is enqueued on the hipStream_t the caller passes (typically
 * torch.cuda.current_stream().cuda_stream); nothing synchronizes the host.
 * The host pipelines (offload / restore) use a `compute` and a `copy` stream
 * and leave the staging buffer free once the stream named in their comment has
 * reached the point of return; a later call that reuses the same staging buffer
 * on other streams must first be ordered after that point.
 * The library must run on the HIP runtime the caller's streams belong to:
 * load it into a process after that runtime (e.g. after `import torch`).
 */
#ifndef IEKV_H_
#define IEKV_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IEKV_ABI_VERSION 21

enum {
  IEKV_OK = 0,
  IEKV_ERR_INVALID = -1, /* bad argument (null pointer, size, alignment, overlap) */
  IEKV_ERR_HIP = -2,     /* a HIP runtime call failed */
  IEKV_ERR_CAPACITY = -3, /* a buffer is too small for the requested blocks */
  IEKV_ERR_RANGE = -4,   /* a host block id outside its pool (the *_ids entry points) */
  IEKV_ERR_IDS = -5,     /* host ids that conflict: a destination block twice in one call,
                            or a copy within one pool whose sources overlap its destinations */
  IEKV_ERR_TIMEOUT = -6  /* iekv_queue_wait: the requests did not finish in time */
};

/* Opaque handle describing one paged pool: the base address of each of its
 * 2L arrays, the tile size and the number of blocks. Registering a pool once
 * replaces the reference's per-call walk over the `k_caches`/`v_caches` lists
 * that LayeredSlotCopier keeps (ie/engine/copier.py:7-12). */
typedef struct iekv_pool iekv_pool;

/* ABI version of the loaded library (IEKV_ABI_VERSION). */
int iekv_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* iekv_last_error(void);

/* Register a pool. `array_ptrs` is a HOST array of n_arrays device addresses
 * (K arrays then V arrays), each array holding num_blocks tiles of tile_bytes.
 * If the arrays are equally spaced (one slab) the handle stores base+stride;
 * otherwise the address table is uploaded once to `device`.
 * Replaces: LayeredSlotCopier.__init__ (ie/engine/copier.py:7-12). */
int iekv_pool_create(const uint64_t* array_ptrs, int32_t n_arrays, int64_t tile_bytes,
                     int64_t num_blocks, int32_t device, iekv_pool** out);

/* Release a pool handle (not the arrays it describes). */
int iekv_pool_destroy(iekv_pool* pool);

/* Direct pool-to-pool handoff: for i < n_blocks and every array a, copy tile
 * src_ids[i] of src array a onto tile dst_ids[i] of dst array a. No staging.
 * Both pools must have the same n_arrays and tile_bytes.
 * Replaces: the composition of disaggregated.py:50 (read_block per src block)
 * and disaggregated.py:81-82 (write_block per dst block), i.e. copier.py:18-31
 * without materialising the payloads. */
int iekv_copy_direct(const iekv_pool* src, const iekv_pool* dst, const int32_t* src_ids,
                     const int32_t* dst_ids, int32_t n_blocks, hipStream_t stream);

/* Fused multi-layer pack (gather): staging[i][a] = tile src_ids[i] of array a.
 * `staging` is device memory of at least n_blocks*n_arrays*tile_bytes bytes.
 * Replaces: `[copier.read_block(b) for b in seq.block_table]`
 * (ie/serve/disaggregated.py:50 over ie/engine/copier.py:18-22). */
int iekv_pack(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
              void* staging, int64_t staging_bytes, hipStream_t stream);

/* Unpack (scatter): tile dst_ids[i] of array a = staging[i][a].
 * Replaces: `for block_id, payload in zip(...): copier.write_block(...)`
 * (ie/serve/disaggregated.py:81-82 over ie/engine/copier.py:24-31), and the
 * single-block restore write (ie/core/block_manager.py:162). */
int iekv_unpack(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                const void* staging, int64_t staging_bytes, hipStream_t stream);

/* Several independent direct handoffs in one call, one launch per request, as a
 * decode step admits several prefilled requests: request k moves counts[k]
 * (host array) blocks, its ids following request k-1's in src_ids / dst_ids
 * (device memory, as iekv_copy_direct takes them), on streams[k % n_streams].
 * When done_events is not null, done_events[k] (created by the caller) is
 * recorded on that stream right after request k's launch, so a consumer can
 * wait for exactly that request. Requests must not share destination blocks.
 * The caller orders every stream after the writes of the source blocks, and
 * waits on the streams or events before reading a destination. Each request's
 * launch is iekv_copy_direct's, issued without a call per request from the
 * caller: the host's cost per request is then HIP's own launch cost (measured
 * 2.3-4.5 us on MI355X boxes, against 0.3 us more through a Python loop).
 * Replaces: the per-prompt handoffs of DisaggregatedEngine.generate
 * (ie/serve/disaggregated.py:106-116), each of them disaggregated.py:50 + :81-82. */
int iekv_copy_direct_requests(const iekv_pool* src, const iekv_pool* dst, int32_t n_requests,
                              const int32_t* counts, const int32_t* src_ids,
                              const int32_t* dst_ids, const hipStream_t* streams,
                              int32_t n_streams, hipEvent_t* done_events);

/* Most block ids one launch of a host-id call (the *_ids entry points below)
 * carries in its kernel arguments. */
#define IEKV_INLINE_IDS 256

/* The same three moves with the block ids given in HOST memory, any number of
 * them: the ids travel in the launches' own kernel arguments, IEKV_INLINE_IDS
 * blocks per launch (a longer list is issued as consecutive launches), so the
 * caller needs no device id buffer and no host-to-device id copy sits on the
 * stream between launches. A launch whose ids fill at most 64 words (32 direct
 * pairs, or 64 pack or unpack ids) carries them in a 256-byte block, a longer
 * one in a 2 KiB block: the runtime copies each launch's arguments on the host,
 * so short lists launch faster. One block per workgroup whatever iekv_set_launch's
 * run_blocks. The ids are checked on the host before anything
 * is enqueued: an id outside its pool returns IEKV_ERR_RANGE; a destination id
 * given twice (iekv_copy_direct_ids, iekv_unpack_ids), or a copy within one pool
 * whose sources overlap its destinations, returns IEKV_ERR_IDS ("one pool": two
 * handles over the same arrays count as one; a source and a destination pool
 * that overlap in memory otherwise return IEKV_ERR_INVALID). iekv_copy_direct_ids
 * issues its (src, dst) pairs in ascending destination order (the pairs are
 * independent; neighbouring destination tiles are then written together).
 * Replace: the same reference lines as iekv_copy_direct, iekv_pack and
 * iekv_unpack, for the per-request calls of the disaggregation workers
 * (ie/serve/disaggregated.py:50, 81-82), whose tables are host lists. */
int iekv_copy_direct_ids(const iekv_pool* src, const iekv_pool* dst, const int32_t* src_ids,
                         const int32_t* dst_ids, int32_t n_blocks, hipStream_t stream);
int iekv_pack_ids(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks, void* staging,
                  int64_t staging_bytes, hipStream_t stream);
int iekv_unpack_ids(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                    const void* staging, int64_t staging_bytes, hipStream_t stream);

/* Slot scatter of one layer's new K/V rows: row i of k (and of v), each
 * tile_bytes/block_size bytes, contiguous [n_tokens][row], lands in row
 * slots[i] (int64, device memory) of K array `layer` (and V array L+layer).
 * Rows whose slot is outside the pool are skipped.
 * Replaces: write_kv, `k_cache[slots] = k` (ie/kernels/reference.py:45-51) /
 * `index_copy_` (ie/kernels/torch_backend.py:13-16). */
int iekv_write_slots(const iekv_pool* pool, int32_t layer, int32_t block_size, const void* k,
                     const void* v, const int64_t* slots, int32_t n_tokens, hipStream_t stream);

/* Paged gather of one array's context: out row j (j < context_len) = row
 * block_table[j / block_size] * block_size + j % block_size of array `array`;
 * out is [context_len][row] bytes (out_bytes checked), block_table int32 in
 * device memory. Rows of out-of-range blocks are left untouched.
 * Replaces: gather_context (ie/kernels/reference.py:54-63,
 * ie/kernels/torch_backend.py:19-24). */
int iekv_gather_rows(const iekv_pool* pool, int32_t array, int32_t block_size,
                     const int32_t* block_table, int32_t context_len, void* out,
                     int64_t out_bytes, hipStream_t stream);

/* write_kv for several layers in one launch: for l < n_layers, row i of layer
 * l of k (and of v), each tile_bytes/block_size bytes at k + l * layer_stride +
 * i * row bytes, lands in row slots[i] (int64, device memory) of K array
 * first_layer + l (and of V array L + first_layer + l). Rows whose slot is
 * outside the pool are skipped. layer_stride may be 0 (every layer takes the
 * same rows).
 * Replaces: the reference's write_kv call in each layer's forward
 * (ie/kernels/reference.py:45-51 / ie/kernels/torch_backend.py:13-16, called
 * once per layer from ie/model/transformer.py:105-110), n_layers calls at once. */
int iekv_write_slots_layers(const iekv_pool* pool, int32_t first_layer, int32_t n_layers,
                            int32_t block_size, const void* k, const void* v,
                            int64_t layer_stride, const int64_t* slots, int32_t n_tokens,
                            hipStream_t stream);

/* gather_context for several arrays in one launch: out is [n_arrays][context_len]
 * [row] bytes (out_bytes checked); its slab y holds the context of array
 * first_array + y, row j = row block_table[j / block_size] * block_size +
 * j % block_size of that array. Rows of out-of-range blocks are left untouched.
 * Replaces: the reference's gather_context calls for the K and V cache of every
 * layer (ie/kernels/reference.py:54-63, ie/kernels/torch_backend.py:19-24, once
 * per array per layer in paged attention), n_arrays calls at once. */
int iekv_gather_rows_arrays(const iekv_pool* pool, int32_t first_array, int32_t n_arrays,
                            int32_t block_size, const int32_t* block_table, int32_t context_len,
                            void* out, int64_t out_bytes, hipStream_t stream);

/* Most bytes of block images one direct host launch moves: offloads and
 * restores whose host range lies in one pinned allocation mapped for the device
 * are moved by the pack / unpack kernel itself (it writes or reads the host
 * buffer), whatever their size, in launches of at most this many bytes of
 * images (one image per launch when a single image is larger); pageable memory
 * goes through the staging buffer. */
#define IEKV_HOST_DIRECT_MAX_BYTES (64LL << 20)

/* Offload to host: pack the blocks chunk by chunk into the device staging
 * buffer (two slots when it holds at least two blocks, else one) on
 * `compute`, and copy each packed chunk to host_dst with hipMemcpyAsync on
 * `copy`, so the pack of chunk k+1 overlaps the device-to-host copy of chunk
 * k. host_dst receives the block-major image [n_blocks][2L][T]. An image whose
 * host range lies in one pinned allocation mapped for the device, of any size,
 * skips the staging buffer: the pack kernel writes host_dst itself, on
 * `compute`, in launches of at most IEKV_HOST_DIRECT_MAX_BYTES of images, and
 * `staging` may then be null (measured on MI355X: 54.4 GB/s in every round on a
 * box where the staged pipeline's runtime copies moved 32-33 GB/s). Pageable
 * memory is staged, which needs at least one block image of staging
 * (IEKV_ERR_CAPACITY otherwise).
 * On return `compute` is ordered after every copy (so the staging
 * buffer and host_dst are free / complete once `compute` reaches that point).
 * `copy` may equal `compute`.
 * Replaces: the payload read of the offload hook,
 * `tier.admit(hash, tokens, copier.read_block(id))` (ie/core/block_manager.py:82),
 * batched over many blocks. */
int iekv_offload(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                 void* host_dst, int64_t host_bytes, void* staging, int64_t staging_bytes,
                 hipStream_t compute, hipStream_t copy);

/* Size of the device staging buffer iekv_offload_static uses (32 MiB), held by
 * the library on every GPU it runs on until the process ends. */
#define IEKV_STATIC_STAGING_BYTES (32LL << 20)

/* Allocation-free offload: iekv_offload with the staging buffer taken from a
 * buffer of IEKV_STATIC_STAGING_BYTES the library holds in each device's
 * memory (two slots when it holds two block images, else one), and with
 * HIP events created once per device; the call itself allocates nothing. The
 * first call on a device sets that device's buffer address and events up.
 * A block image (2L * T bytes) larger than IEKV_STATIC_STAGING_BYTES is
 * rejected with IEKV_ERR_CAPACITY before anything is enqueued. Every call on
 * one device shares that device's buffer and events. Calls are enqueued one at
 * a time (a lock is held while a call enqueues its work, so calls from several
 * host threads wait for each other), and a call that uses the buffer makes its
 * `compute` stream wait for the previous such call's last device-to-host copy:
 * calls on unrelated streams, or from other threads, never overwrite a slot
 * an earlier call still copies from. The buffer keeps the last call's bytes;
 * nothing in it needs to start at zero. Streams, host image and ordering on
 * return as for iekv_offload.
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory or call allocating routines (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); it runs the
 * kernels of iekv_offload. */
int iekv_offload_static(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                        void* host_dst, int64_t host_bytes, hipStream_t compute,
                        hipStream_t copy);

/* Restore from host onto dst_ids. An image whose host range lies in one pinned
 * allocation mapped for the device, of any size, is read by the unpack kernel
 * itself on `compute`, in launches of at most IEKV_HOST_DIRECT_MAX_BYTES of
 * images: measured on MI355X this held 52-57 GB/s in every state of the box,
 * where runtime copies of the same images ran at 28-56 GB/s. Otherwise (pageable
 * memory) chunk k of host_src is copied into a staging slot with hipMemcpyAsync
 * on `copy` while `compute` unpacks chunk k-1; that path needs a staging buffer
 * of at least one block image (IEKV_ERR_CAPACITY otherwise), the direct one none
 * (`staging` may be null). On return `copy` is ordered after the last
 * unpack, so the staging buffer and host_src may be reused by later work on
 * either stream.
 * Replaces: the restore write of a tier hit, `copier.write_block(block.id,
 * entry[1])` (ie/core/block_manager.py:159-162), batched over many blocks. */
int iekv_restore(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                 const void* host_src, int64_t host_bytes, void* staging, int64_t staging_bytes,
                 hipStream_t compute, hipStream_t copy);

/* Most images iekv_restore_blocks restores directly from pinned host memory
 * in one launch (their addresses ride in the kernel arguments). */
#define IEKV_INLINE_IMAGES 128

/* Restore from scattered host images: like iekv_restore, but block i's image
 * ([2L][T] bytes) is read from host_blocks[i], a HOST array of n_blocks host
 * addresses. When every image lies in pinned host memory mapped for the device,
 * the unpack kernel reads them itself on `compute`, up to IEKV_INLINE_IMAGES
 * images and IEKV_HOST_DIRECT_MAX_BYTES per launch, their addresses in the
 * kernel arguments, and `staging` may be null. Otherwise they go through the
 * staging buffer (at least one block image), and images that are adjacent in
 * host memory within one allocation are copied together.
 * On return `copy` is ordered after the last unpack, as for iekv_restore.
 * Replaces: the restore loop of a prefix plan's tier hits,
 * `for key in offloaded: ... copier.write_block(block.id, payload)`
 * (ie/core/block_manager.py:159-167), whose payloads the tier took one by one
 * and which therefore live at unrelated host addresses, as one call. */
int iekv_restore_blocks(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                        const void* const* host_blocks, void* staging, int64_t staging_bytes,
                        hipStream_t compute, hipStream_t copy);

/* The offload with one host image per block: block src_ids[i] is packed into
 * the image at host_blocks[i] ([2L][T] bytes, a HOST array of n_blocks
 * addresses), so each image can live in its own allocation and be freed on its
 * own. When every image is in pinned memory mapped for the device, pack
 * launches on `compute` write them, up to IEKV_INLINE_IMAGES images and
 * IEKV_HOST_DIRECT_MAX_BYTES per launch, the addresses in the kernel arguments,
 * and `staging` may be null; otherwise chunks are packed into `staging` (at
 * least one block image) and copied to the host on `copy` (one hipMemcpyAsync
 * per run of images adjacent within one allocation), as iekv_offload does.
 * Replaces: the same payload reads as iekv_offload
 * (`copier.read_block(id)` in the offload hook, ie/core/block_manager.py:82),
 * for a tier that keeps each block's payload on its own. */
int iekv_offload_blocks(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                        void* const* host_blocks, void* staging, int64_t staging_bytes,
                        hipStream_t compute, hipStream_t copy);

/* The host-tier calls above with their block ids in HOST memory, any
 * number of them, as the *_ids handoff calls take theirs: the ids are checked
 * first (IEKV_ERR_RANGE for an id outside the pool; for the restores,
 * IEKV_ERR_IDS for a destination given twice), then travel in the launches'
 * own kernel arguments, so no id upload precedes the move on the stream.
 * Otherwise each behaves exactly as the call it mirrors.
 * Replace: the same reference lines as iekv_offload, iekv_restore,
 * iekv_restore_blocks and iekv_offload_blocks, for callers whose block lists
 * are host-side (the block manager's tables). */
int iekv_offload_ids(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                     void* host_dst, int64_t host_bytes, void* staging, int64_t staging_bytes,
                     hipStream_t compute, hipStream_t copy);
int iekv_restore_ids(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                     const void* host_src, int64_t host_bytes, void* staging,
                     int64_t staging_bytes, hipStream_t compute, hipStream_t copy);
int iekv_restore_blocks_ids(const iekv_pool* dst, const int32_t* dst_ids, int32_t n_blocks,
                            const void* const* host_blocks, void* staging,
                            int64_t staging_bytes, hipStream_t compute, hipStream_t copy);
int iekv_offload_blocks_ids(const iekv_pool* src, const int32_t* src_ids, int32_t n_blocks,
                            void* const* host_blocks, void* staging, int64_t staging_bytes,
                            hipStream_t compute, hipStream_t copy);

/* Pinned host memory of exactly `bytes` bytes, mapped for every GPU
 * (hipHostMalloc), for host images the calls above read or write directly:
 * *out receives its address, or null with IEKV_ERR_HIP and the runtime's
 * message when the memory cannot be had. iekv_host_free returns it (null is a
 * no-op); no copy may still use it then. Allocators that round requests up (a
 * caching allocator rounding to powers of two pins 4 MiB for a 2.5 MiB block
 * image, 64 GiB for a 43 GB one) pin up to twice what the images need.
 * Replaces: the host arrays the reference's payloads and tier entries live in
 * (`.copy()` of each tile, ie/engine/copier.py:21-22; KVTier entries,
 * ie/core/offload.py:26-69), page-locked so the GPU reaches them. */
int iekv_host_alloc(int64_t bytes, void** out);
int iekv_host_free(void* ptr);

/* Launch floor, for measurement: `launches` launches of an empty kernel of
 * `workgroups` workgroups of 256 lanes on `stream`, dispatched as the move
 * kernels are (timed by iekv_profile_start like them). The in-dispatch time
 * of one launch is what any launch costs before it moves a byte; the host time
 * of the call over `launches` is the host's cost of issuing one.
 * No reference counterpart: a measurement aid. */
int iekv_noop(int32_t workgroups, int32_t launches, hipStream_t stream);

/* Launch shape of the move kernels (process-wide):
 *   run_blocks  blocks per workgroup run, 1..64; 0 = automatic (currently one
 *               block per workgroup); -1 keeps the current setting;
 *   unroll      16-byte accesses in flight per lane per step: 1, 2, 4, 8 or
 *               16 (capped by what a chunk needs); 0 keeps the current setting;
 *   nontemporal 1 for streaming (non-temporal) loads and stores, 0 for
 *               ordinary ones, -1 keeps the current setting; a pack that
 *               writes pinned host memory itself (a direct offload) uses
 *               ordinary ones for tiles of 16 KiB or more either way;
 *   order       which (array, block) tiles are in flight together in the
 *               launches that write a pool (direct copy, unpack, restore):
 *               0 array-major (the 2L tiles of one block), 1 block-major
 *               (random blocks of one array), 2 diagonal (array a takes list
 *               run r + a, so 2L arrays and 2L blocks at once), 3 scattered
 *               (the (array, block) pairs in a multiplicative-hash order over
 *               the whole move); adding 4
 *               gives each of the 8 XCDs one contiguous share of that order
 *               (with 5, its own eighth of the arrays); -1 keeps the current
 *               setting;
 *   pack_order  the same choice for the launches that write a staging buffer
 *               (pack, offload);
 *   chunk_bytes with one block per workgroup, each tile is split into a
 *               power-of-two number of chunks of at least this many bytes,
 *               one workgroup per chunk (the chunks of one tile are adjacent
 *               in the order); a tile smaller than this whose 16-byte (or
 *               narrower) vectors divide 256 lanes is grouped instead: one
 *               workgroup moves a block's tiles in chunk_bytes / tile_bytes
 *               consecutive arrays; 0 moves one whole tile per workgroup; a
 *               power of two from 64 to 1 MiB; -1 keeps the current setting.
 *               A launch that would exceed the dispatch limit of 2^32 - 1
 *               work-items halves the split, then spreads over several
 *               launches. This sets the chunk size of every move, the
 *               launches that write a pool included (iekv_set_direct_chunk
 *               sets theirs alone), except the unpacks that read pinned host
 *               memory themselves (direct restores), which move whole tiles,
 *               or groups of tiles smaller than this size.
 * The defaults (run 0, unroll 8, nontemporal 1, order, pack_order and
 * chunk_bytes 4096 for the launches that write a staging image; 8192 for the
 * launches that write a pool, iekv_set_direct_chunk) are the library's measured
 * best; iekv_get_launch and iekv_get_direct_chunk report them.
 * No reference counterpart: a tuning knob for the launches the entry points
 * above make. */
int iekv_set_launch(int32_t run_blocks, int32_t unroll, int32_t nontemporal, int32_t order,
                    int32_t pack_order, int32_t chunk_bytes);

/* Per-launch timing, for measurement (calling thread only). After
 * iekv_profile_start(max_launches), each of the next max_launches kernel
 * launches made by the entry points above carries a start/stop event pair in
 * its own dispatch (hipExtLaunchKernelGGL), so timing adds no packets to the
 * stream. iekv_profile_stop waits for the last timed launch, writes up to
 * `capacity` durations in launch order to durations_ms, stores the number of
 * timed launches in *count and ends the session.
 * No reference counterpart: the reference times nothing below Python's
 * perf_counter (ie/bench/harness.py:67-120). */
int iekv_profile_start(int32_t max_launches);
int iekv_profile_stop(float* durations_ms, int32_t capacity, int32_t* count);

/* Bits iekv_check_ids writes to *status (0 = every check passed). */
#define IEKV_IDS_SRC_RANGE 1    /* a source id outside [0, num_blocks) of its pool */
#define IEKV_IDS_DST_RANGE 2    /* a destination id outside its pool */
#define IEKV_IDS_DST_REPEATED 4 /* a destination id given more than once */
#define IEKV_IDS_OVERLAP 8      /* src == dst and a block is both a source and a destination */

/* Bytes of workspace iekv_check_ids needs for a destination pool of num_blocks:
 * one bit per block, in 32-bit words. */
#define IEKV_CHECK_WORKSPACE_BYTES(num_blocks) ((((int64_t)(num_blocks)) + 31) / 32 * 4)

/* Check a list of block ids held in DEVICE memory on the GPU, as the host-id
 * calls check theirs on the host, before a call that takes the list (in stream
 * order, so the check sees the ids that call will read). Either pool may be
 * null: with src, src_ids[0..n_blocks) are checked against src's size; with
 * dst, dst_ids are checked against dst's size and for repeats; with src == dst,
 * also that no block is both a source and a destination (a direct copy within
 * one pool). `workspace` is device memory of at least
 * IEKV_CHECK_WORKSPACE_BYTES(dst->num_blocks) bytes (none without dst);
 * `status` is one device int32, overwritten with the IEKV_IDS_* bits of the
 * failed checks. Pools are compared by the memory they describe: two handles
 * over the same arrays count as one pool, and pools whose arrays overlap
 * otherwise are refused (IEKV_ERR_INVALID). Two or three small launches on `stream`, no host
 * synchronisation: the caller reads *status after the stream has passed them
 * (and may skip the move, or read it after the move, to report). The launches
 * are not timed by iekv_profile_start. Calls that share a workspace or status
 * word must be ordered on one stream.
 * No reference counterpart: the reference's copier slices its caches one block
 * at a time (ie/engine/copier.py:14-31) and checks no id; this gives callers
 * that keep ids on the device the checks the host-id calls make. */
int iekv_check_ids(const iekv_pool* src, const int32_t* src_ids, const iekv_pool* dst,
                   const int32_t* dst_ids, int32_t n_blocks, void* workspace,
                   int64_t workspace_bytes, int32_t* status, hipStream_t stream);

/* Current launch shape, for reporting. */
int iekv_get_launch(int32_t* run_blocks, int32_t* unroll, int32_t* nontemporal,
                    int32_t* order, int32_t* pack_order, int32_t* chunk_bytes);

/* chunk_bytes of iekv_set_launch for the launches that write a pool from HBM
 * alone: pool-to-pool moves (iekv_copy_direct, iekv_copy_direct_ids and
 * iekv_copy_direct_requests) and, since ABI 20, unpacks of a device or
 * pageable-host staging image (iekv_unpack, iekv_unpack_ids, the staged
 * restores) whose tiles are at least this large; unpacks of smaller tiles keep
 * the staging chunk, which groups them as the pack does. The same values and
 * meaning; -1 keeps the current setting. iekv_get_direct_chunk reports it
 * (chunk_bytes of iekv_get_launch is the setting of the launches that write a
 * staging image).
 * No reference counterpart: a tuning knob, like iekv_set_launch. */
int iekv_set_direct_chunk(int32_t chunk_bytes);
int iekv_get_direct_chunk(int32_t* chunk_bytes);

/* ---- Request queue: per-request direct handoffs without a launch each ----
 *
 * A queue serves direct handoffs (iekv_copy_direct_ids's move) between one
 * source and one destination pool through a resident kernel, so a request costs
 * the host a descriptor write instead of a kernel launch. The kernel (one
 * leader workgroup and `workers` mover workgroups) reads descriptors from a
 * ring in pinned host memory, copies them to device memory, and the movers
 * claim each request's tiles a few at a time; the last mover to finish a
 * request writes its completion to the ring, where iekv_queue_wait reads it.
 *
 * Every wait of the kernel is bounded: it ends after iekv_queue_stop, after
 * `idle_us` without a new request, or `life_us` after it started, whichever
 * comes first. The library restarts it by itself (a stop that drains every
 * request already submitted, then one launch) before a submission when the
 * last one is more than idle_us / 2 old, or the kernel more than life_us / 2,
 * so a submitted request is never left to a kernel that may already have ended.
 *
 * Ordering. Requests are moved as soon as they are submitted, independently of
 * every stream: the caller submits only requests whose source blocks are
 * written (e.g. after synchronizing the stream that wrote them), and reads a
 * destination only after iekv_queue_wait (or iekv_queue_poll) reports its
 * ticket done. Requests in flight together must not share destination blocks,
 * nor write blocks another one reads. Each request's ids are checked as
 * iekv_copy_direct_ids checks them. Calls on one queue are serialized by a
 * lock; the pools must outlive the queue. While it runs, the kernel holds
 * workers + 1 workgroups resident (by default one per compute unit), so other
 * kernels share the GPU with it; hipDeviceSynchronize
 * and hipFree wait for it to end (iekv_queue_stop ends it at once).
 *
 * No reference counterpart: the reference hands off one request at a time
 * (DisaggregatedEngine.generate, ie/serve/disaggregated.py:106-116, each a
 * disaggregated.py:50 read + :81-82 write); this serves that call pattern for
 * requests of a few MB, whose launches otherwise cost more than their bytes. */
typedef struct iekv_queue iekv_queue;

/* Descriptors in flight at once (a submission waits for the one IEKV_QUEUE_SLOTS
 * earlier to finish), and blocks per descriptor (a longer request is split into
 * several descriptors; its ticket is that of the last). */
#define IEKV_QUEUE_SLOTS 256
#define IEKV_QUEUE_MAX_BLOCKS 1024
/* Ticket of an empty request: already done. */
#define IEKV_QUEUE_DONE UINT64_MAX

/* Make a queue for direct handoffs from `src` to `dst` (same n_arrays and
 * tile_bytes, one device). workers: mover workgroups, each wave of which is a
 * mover (0: one per compute unit, the leader's workgroup included);
 * claim_bytes: most bytes one mover claims at once (0: 512 KiB); idle_us /
 * life_us: the kernel's idle and lifetime limits (0: 200 ms / 60 s). Allocates
 * the rings (about 2 MiB of pinned host memory, 11 MiB of device memory) and a
 * stream; launches nothing until the first submission. */
int iekv_queue_create(const iekv_pool* src, const iekv_pool* dst, int32_t workers,
                      int64_t claim_bytes, int64_t idle_us, int64_t life_us,
                      iekv_queue** out);

/* Submit one request: tile src_ids[i] of every array onto tile dst_ids[i]
 * (HOST memory, n_blocks of each, checked first). *ticket identifies it for
 * iekv_queue_wait / iekv_queue_poll (tickets grow by one per descriptor over
 * the queue's life); n_blocks == 0 gives IEKV_QUEUE_DONE. */
int iekv_queue_submit(iekv_queue* q, const int32_t* src_ids, const int32_t* dst_ids,
                      int32_t n_blocks, uint64_t* ticket);

/* Submit n_requests requests in one call, as iekv_queue_submit would one after
 * another: request k moves counts[k] blocks, its ids following request k-1's in
 * src_ids / dst_ids (HOST memory); tickets[k] receives its ticket. Every request
 * is checked before any is submitted. */
int iekv_queue_submit_requests(iekv_queue* q, int32_t n_requests, const int32_t* counts,
                               const int32_t* src_ids, const int32_t* dst_ids,
                               uint64_t* tickets);

/* Wait until every request up to and including `ticket` is done, or return
 * IEKV_ERR_TIMEOUT after timeout_us (< 0: 10 s). IEKV_ERR_INVALID for a ticket
 * not issued yet. */
int iekv_queue_wait(iekv_queue* q, uint64_t ticket, int64_t timeout_us);

/* *done = 1 when every request up to and including `ticket` is done, else 0. */
int iekv_queue_poll(iekv_queue* q, uint64_t ticket, int32_t* done);

/* Finish every submitted request, end the kernel and wait for it to exit.
 * The next submission starts it again. */
int iekv_queue_stop(iekv_queue* q);

/* Stop the queue and release it. */
int iekv_queue_destroy(iekv_queue* q);

/* Counters of a queue: requests (descriptors) served, kernel launches (sessions). */
int iekv_queue_stats(const iekv_queue* q, uint64_t* descriptors, uint64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* IEKV_H_ */
