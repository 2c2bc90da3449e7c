"""KV-cache handoff benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg3] [--seed 0]

A step is one full handoff of the workload: every request's blocks move from
the prefill pool to the decode pool under the destination ids a decode
worker's BlockManager hands out (iekv.workloads). Both pools are resident in
HBM before timing starts, carved from one allocation with the prefill pool first
(iekv.engine.pools.allocate_pool_pair, as DisaggregatedEngine allocates them;
--separate-pools allocates them apart); the src pool holds N(0,1) values (raw random bytes
without NaN codes for fp8). Legs:

  direct       one iekv_copy_direct launch per request (the headline: 2P bytes); like
               every per-request leg, consecutive requests alternate between --streams
               streams, so one request's launch can start while the previous one drains
               (default: two when the workload's median request moves at most 512 MiB
               each way, else one; see OVERLAP_MAX_REQUEST_BYTES)
  pack_unpack  iekv_pack into a per-request staging buffer, then iekv_unpack (4P bytes)
  pack         the pack half alone (2P bytes); unpack: the unpack half alone (2P bytes)
  batched      all requests' blocks in ONE direct launch (2P bytes)
  direct_ids   the direct leg with each request's table in host memory
               (iekv_copy_direct_ids: ids checked on the host, carried in the launch's
               kernel arguments)
  copier       the drop-in Python path: HipSlotCopier.copy_blocks per request with the
               block tables as Python lists (id checks and hand-over included; 2P bytes)
  copier_pack_unpack  the same for pack mode: read_blocks then write_blocks (4P bytes)
  requests     the direct leg's per-request launches issued by the library in one call
               per step (iekv_copy_direct_requests), without a Python loop (2P bytes)
  write_kv     the prefill side: every request's new K/V rows of every layer scattered
               into the prefill pool by slot, one iekv_write_slots_layers launch per
               request (read + write of every row); write_kv_per_layer: one
               iekv_write_slots launch per request and layer, as the reference calls
               write_kv once per layer
  gather_context  the decode side: every request's context gathered from every K and V
               array of the decode pool through its block table (resident prefix
               included), one iekv_gather_rows_arrays launch per request (read + write
               of every row); gather_per_array: one iekv_gather_rows launch per request
               and array, as the reference calls gather_context once per cache
  queue        the direct handoffs served by the resident request queue
               (iekv.engine.queue.HandoffQueue): each step's requests submitted with one
               library call (iekv_queue_submit_requests, one descriptor and ticket per
               request), then the last ticket waited for; timed by the host clock from
               the first submission to the last completion (2P bytes). Also reports each
               request's latency, submitted and waited for alone (ms_per_request), beside
               that of one direct launch per request with a stream synchronize after it
               (launch_latency_ms), measured before the queue's kernel starts
  queue_py     the same with one HandoffQueue.submit call per request from Python
  host_roundtrip  every moved block offloaded to pinned host memory with one iekv_offload
               and restored with one iekv_restore (host-link bound), then the same
               calls once per block on up to 1,024 blocks, then the drop-in tier path

``value`` is the direct leg's algorithmic read+write bandwidth, 2P / step
time, in GB/s (P = blocks x 2L x T); the step time comes from two HIP events
around the timed steps on the launch stream, which every request stream joins
at the end of a step, with nothing else added between launches.
``roofline.achieved`` is the algorithmic bytes per kv_move launch divided by
the average launch duration, measured in a second timed pass over the same
steps, one launch at a time on the launch stream, by HIP events that ride in
each launch's own dispatch packet (iekv_profile_start /
hipExtLaunchKernelGGL); ``ms_per_request`` comes from the same pass. After timing, every destination
tile is compared with its source tile on the GPU (the whole workload, bit for
bit). ``cpu_baseline`` times the NumPy restatement of the reference handoff
(oracle/) on a bounded sample of the same shape on this host, single-threaded.
"""
from __future__ import annotations

import argparse
import faulthandler
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "inference-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
# HBM bytes per algorithmic byte of the direct kv_move launches on cfg3 with the
# library's default launch shape, from two rocprofv3 --pmc runs (FETCH_SIZE, then
# WRITE_SIZE) calibrated on a plain 4 GiB copy; the summary states the command and
# ends with a "traffic_ratio <x>" line. Used only for the configuration it measured.
PMC_SUMMARY = ROOT / "profiles" / "kv_move_direct_cfg3_pmc.txt"
# Names of the cache dtypes in the bench line (the kernels move their raw bits).
DTYPE_NAMES = {"float32": "f32", "float16": "f16", "bfloat16": "bf16", "fp8_e4m3": "fp8_e4m3",
               "uint8": "u8"}
METRIC = "KV handoff GB/s (read+write) and % of HBM peak; ms per request handoff"
# Legs that move the workload's blocks from the prefill pool to the decode pool; the
# first of them in --legs gives the line's value (2P / step time).
HANDOFF_LEGS = ("direct", "pack_unpack", "pack", "unpack", "batched", "copier",
                "copier_pack_unpack", "requests", "direct_ids", "queue", "queue_py")
# Legs served by the resident request queue: timed by the host clock (the kernel runs
# for the whole pass, so there are no launches to time), the queue stopped after them.
QUEUE_LEGS = ("queue", "queue_py")
# The slot kernels on either side of the handoff (prefill's KV writes, decode's reads).
SLOT_LEGS = ("write_kv", "write_kv_per_layer", "gather_context", "gather_per_array")
# Requests of up to this many payload bytes (one direction) overlap on two request
# streams: one launch's drain and the next one's ramp-up (about 5 us) then run at the
# same time. Longer launches gain less from that than two concurrent scattered moves
# lose to each other. Measured in one process per workload, one stream against two:
# requests of 33-508 MiB (the 8B shape and its tp=2/tp=8 shares) gained 1-12% on the
# direct leg from two; requests of 640 MiB to 2.5 GiB (the 70B share at tp=4, tp=2 and
# whole) ran every leg faster on one: direct +0.3-1.6%, pack +1.8-4.5%, unpack
# +1.3-3.5%, pack -> unpack +2.4-3.0%.
OVERLAP_MAX_REQUEST_BYTES = 512 << 20


def request_streams(w) -> int:
    """Request streams for a workload's per-request legs: two when its median request
    moves at most OVERLAP_MAX_REQUEST_BYTES each way, else one."""
    sizes = sorted(len(t) * w.shape.block_bytes for t in w.src_tables)
    return 2 if sizes and sizes[len(sizes) // 2] <= OVERLAP_MAX_REQUEST_BYTES else 1


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


DEFAULT_LAUNCH = {"run_blocks": 0, "unroll": 8, "nontemporal": 1, "order": 5, "pack_order": 0,
                  "chunk_bytes": 4096, "direct_chunk_bytes": 8192}


def measured_traffic(config: str, tp: int, leg: str, launch: dict, separate: bool,
                     bytes_per_launch: float) -> tuple[int | None, str]:
    """HBM bytes per launch of the dominant kernel from the committed PMC summary, and
    where that figure comes from. Only the case the summary measured (cfg3, whole
    heads, the direct leg, default launch shape, paired pools) gets a number."""
    if (config, tp, leg, separate) != ("cfg3", 1, "direct", False) or launch != DEFAULT_LAUNCH:
        return None, f"not measured for this case (PMC summary covers cfg3 direct: {PMC_SUMMARY.name})"
    ratio = None
    if PMC_SUMMARY.exists():
        for line in PMC_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_ratio "):
                ratio = float(line.split()[1])
    if ratio is None:
        return None, f"{PMC_SUMMARY.name} holds no traffic_ratio line"
    return int(bytes_per_launch * ratio), (
        f"{PMC_SUMMARY.relative_to(ROOT)}: rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 "
        f"(calibrated on a 4 GiB copy) = {ratio} x the algorithmic bytes per launch")


def torch_dtype(name: str):
    import torch

    return {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
            "fp8_e4m3": torch.float8_e4m3fn, "uint8": torch.uint8}[name]


def fill_pool(arrays, dtype_name: str, seed: int) -> None:
    """N(0,1) values, or uniform random bytes without the e4m3fn NaN codes 0x7F / 0xFF."""
    import torch

    gen = torch.Generator(device=arrays[0].device)
    gen.manual_seed(seed)
    for t in arrays:
        if dtype_name == "fp8_e4m3":
            raw = t.view(torch.uint8)
            r = torch.randint(0, 254, raw.shape, dtype=torch.int16, device=t.device,
                              generator=gen)
            raw.copy_((r + (r >= 0x7F).to(torch.int16)).to(torch.uint8))
        else:
            t.normal_(generator=gen)


def host_roundtrip_plan(workload, sample_blocks: int) -> dict:
    """The pinned host memory the host_roundtrip leg holds, phase by phase.

    The whole-list image is pinned at exactly the payload's size and freed
    before the tier phase, whose one-block buffers (at most two flush groups'
    worth beyond the sample, while the previous round's buffers are released)
    are pinned at exactly one block image each.
    """
    P = workload.payload_bytes
    bb = workload.shape.block_bytes
    tier = (sample_blocks + 2 * 64) * bb
    return {"image_bytes": P, "tier_bytes": tier, "peak_pinned_bytes": max(P, tier)}


def host_memory_budget() -> int | None:
    """Bytes of host memory this process can still take: the smaller of the kernel's
    MemAvailable and the room left under the cgroup's memory limit (None when
    neither can be read)."""
    budget = []
    try:
        for line in Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemAvailable:"):
                budget.append(int(line.split()[1]) * 1024)
    except OSError:
        pass
    for limit_file, usage_file in (("/sys/fs/cgroup/memory.max", "/sys/fs/cgroup/memory.current"),
                                   ("/sys/fs/cgroup/memory/memory.limit_in_bytes",
                                    "/sys/fs/cgroup/memory/memory.usage_in_bytes")):
        try:
            limit = Path(limit_file).read_text().strip()
            usage = int(Path(usage_file).read_text().strip())
        except (OSError, ValueError):
            continue
        if limit.isdigit() and int(limit) < (1 << 60):
            budget.append(int(limit) - usage)
        break
    return min(budget) if budget else None


# Host memory the leg leaves to the rest of the process (Python, torch, the HIP
# runtime's own buffers) on top of what it pins.
HOST_MARGIN_BYTES = 8 << 30


def check_host_budget(plan: dict, budget: int | None) -> None:
    """Raise a clear error when the leg's pinned peak plus a margin exceeds the host
    memory available, instead of pinning into a host that cannot hold it."""
    need = plan["peak_pinned_bytes"] + HOST_MARGIN_BYTES
    if budget is not None and need > budget:
        raise RuntimeError(
            f"host_roundtrip needs {need / 1e9:.1f} GB of host memory "
            f"({plan['peak_pinned_bytes'] / 1e9:.1f} GB pinned + "
            f"{HOST_MARGIN_BYTES / 1e9:.1f} GB margin); {budget / 1e9:.1f} GB is available")


class Legs:
    def __init__(self, workload, device, seed: int, pool_layout: str = "paired",
                 streams: int = 1, pad_blocks: int = 0) -> None:
        import torch

        from iekv.engine.copier import issue_order
        from iekv.engine.pools import KVPool, allocate_pool, allocate_pool_pair

        self.torch = torch
        self.w = workload
        s = workload.shape
        dtype = torch_dtype(s.dtype)
        t0 = time.perf_counter()
        self.pool_layout = pool_layout
        if pool_layout == "paired":
            (self.src_k, self.src_v), (self.dst_k, self.dst_v) = allocate_pool_pair(
                workload.src_pool_blocks, workload.dst_pool_blocks, s.block_size, s.layers,
                s.kv_heads, s.head_dim, dtype=dtype, device=device, zero=False,
                pad_blocks=pad_blocks)
            fill_pool(self.src_k + self.src_v, s.dtype, seed)
            for t in self.dst_k + self.dst_v:
                t.zero_()
        else:
            self.src_k, self.src_v = allocate_pool(workload.src_pool_blocks, s.block_size,
                                                   s.layers, s.kv_heads, s.head_dim, dtype=dtype,
                                                   device=device, zero=False,
                                                   pad_blocks=pad_blocks)
            fill_pool(self.src_k + self.src_v, s.dtype, seed)
            self.dst_k, self.dst_v = allocate_pool(workload.dst_pool_blocks, s.block_size,
                                                   s.layers, s.kv_heads, s.head_dim, dtype=dtype,
                                                   device=device, zero=True,
                                                   pad_blocks=pad_blocks)
        self.src = KVPool(self.src_k, self.src_v, s.block_size)
        self.dst = KVPool(self.dst_k, self.dst_v, s.block_size)
        # pack/unpack move blocks in table order (the payload layout); direct copies
        # issue each request's pairs by destination id, as HipSlotCopier.copy_blocks does.
        self.src_ids = [self.src.block_ids(t) for t in workload.src_tables]
        self.dst_ids = [self.dst.block_ids(t, unique=True) for t in workload.dst_tables]
        pairs = [issue_order(s, d) for s, d in zip(workload.src_tables, workload.dst_tables)]
        self.src_direct = [self.src.block_ids(s) for s, _ in pairs]
        self.dst_direct = [self.dst.block_ids(d, unique=True) for _, d in pairs]
        src_all, dst_all = issue_order(sum(workload.src_tables, []), sum(workload.dst_tables, []))
        self.src_all = self.src.block_ids(src_all)
        self.dst_all = self.dst.block_ids(dst_all, unique=True)
        longest = max(len(t) for t in workload.src_tables)
        self.staging = torch.empty(longest * s.block_bytes, dtype=torch.uint8, device=device)
        self.stream = torch.cuda.current_stream(device)
        # Request k of a per-request leg is issued on stream k mod S (every stream at the
        # default priority), so independent requests' launches can overlap their ramp-up
        # and drain; each stream has its own staging buffer. A step starts with every
        # stream waiting on the launch stream and ends with the launch stream waiting on
        # every other stream, so the step events on the launch stream bracket all work.
        self.streams = [self.stream] + [torch.cuda.Stream(device) for _ in range(streams - 1)]
        self.stagings = [self.staging] + [torch.empty_like(self.staging)
                                          for _ in range(streams - 1)]
        # Random bytes in the staging buffers, so an unpack leg timed before any pack
        # reads data like the pools' (zero-filled memory reads faster on this GPU).
        gen = torch.Generator(device=device)
        gen.manual_seed(seed + 1)
        for st in self.stagings:
            st.copy_(torch.randint(0, 256, st.shape, dtype=torch.uint8, device=device,
                                   generator=gen))
        self.last_streams = 1     # request streams the most recent timed pass used
        self._fork_event = torch.cuda.Event()
        self._join_events = [torch.cuda.Event() for _ in self.streams[1:]]
        self.step_ms: dict[str, list[float]] = {}
        self.issue_ms: dict[str, list[float]] = {}   # host time to issue each timed step
        torch.cuda.synchronize()
        log(f"[bench] pools ready: 2 x {workload.src_pool_blocks} blocks x {s.block_bytes} B "
            f"({2 * workload.src_pool_blocks * s.block_bytes / 1e9:.1f} GB) in "
            f"{time.perf_counter() - t0:.1f} s")

    # -- one step of each leg, and the (bytes, request) of each launch it makes -------------
    def plan(self, name: str) -> list[tuple[int, int]]:
        bb = self.w.shape.block_bytes
        sizes = [len(t) for t in self.w.src_tables]
        if name in ("direct", "requests", *QUEUE_LEGS):
            return [(2 * n * bb, r) for r, n in enumerate(sizes)]
        if name == "pack_unpack":
            return [x for r, n in enumerate(sizes) for x in ((2 * n * bb, r), (2 * n * bb, r))]
        if name == "direct_ids":
            from iekv import _native

            step = _native.INLINE_IDS
            return [(2 * min(step, n - k) * bb, r) for r, n in enumerate(sizes)
                    for k in range(0, n, step)]
        if name in ("copier", "copier_pack_unpack"):
            # the copier hands a table of up to HOST_IDS_MAX ids to the library's
            # host-id entry points, which issue INLINE_IDS ids per launch; a longer
            # table is uploaded and moved in one launch
            from iekv import _native
            from iekv.engine.copier import HOST_IDS_MAX

            def launches(n, r):
                if n > HOST_IDS_MAX:
                    return [(2 * n * bb, r)]
                step = _native.INLINE_IDS
                return [(2 * min(step, n - k) * bb, r) for k in range(0, n, step)]

            per = 2 if name == "copier_pack_unpack" else 1   # pack, then unpack
            return [x for r, n in enumerate(sizes) for _ in range(per) for x in launches(n, r)]
        if name in ("pack", "unpack"):
            return [(2 * n * bb, r) for r, n in enumerate(sizes)]
        if name == "batched":
            return [(2 * sum(sizes) * bb, 0)]
        if name in SLOT_LEGS:
            row = self.w.shape.tile_bytes // self.w.shape.block_size
            L, A = self.w.shape.layers, self.w.shape.n_arrays
            tokens, contexts = self._slot_sizes()
            if name == "write_kv":            # K and V rows of every layer per launch
                return [(4 * n * row * L, r) for r, n in enumerate(tokens)]
            if name == "write_kv_per_layer":  # K and V rows of one layer per launch
                return [(4 * n * row, r) for r, n in enumerate(tokens) for _ in range(L)]
            if name == "gather_context":      # every array's context per launch
                return [(2 * n * row * A, r) for r, n in enumerate(contexts)]
            return [(2 * n * row, r) for r, n in enumerate(contexts) for _ in range(A)]
        return []

    # -- request streams ----------------------------------------------------------------
    def _fork(self) -> list[int]:
        """Order every request stream after the launch stream; their raw handles."""
        if len(self.streams) > 1:
            self._fork_event.record(self.stream)
            for st in self.streams[1:]:
                st.wait_event(self._fork_event)
        return [st.cuda_stream for st in self.streams]

    def _join(self) -> None:
        """Order the launch stream after every request stream."""
        for st, ev in zip(self.streams[1:], self._join_events):
            ev.record(st)
            self.stream.wait_event(ev)

    # -- the slot kernels on either side of the handoff -------------------------------------
    def _slot_sizes(self) -> tuple[list[int], list[int]]:
        """Tokens each request's prefill writes (those of its moved blocks; a resident
        prefix is not written) and the context its decode reads (all its tokens)."""
        bs = self.w.shape.block_size
        tokens = [n - (-(-n // bs) - len(t)) * bs for n, t in zip(self.w.lengths, self.w.src_tables)]
        return tokens, list(self.w.lengths)

    def _slot_inputs(self):
        """Per-request slots (prefill pool), decode block tables (resident prefix first),
        every layer's new K/V rows [L, tokens, H, D] and a context buffer
        [2L, context, H, D]; built once."""
        if not hasattr(self, "_slots"):
            torch = self.torch
            s = self.w.shape
            bs = s.block_size
            dev = self.src_k[0].device
            tokens, contexts = self._slot_sizes()
            slots, tables = [], []
            for n, src_t, dst_t in zip(tokens, self.w.src_tables, self.w.dst_tables):
                pos = torch.arange(n, device=dev)
                table = torch.tensor(src_t, dtype=torch.int64, device=dev)
                slots.append((table[pos // bs] * bs + pos % bs).contiguous())
                tables.append(torch.tensor(list(self.w.resident_prefix) + list(dst_t),
                                           dtype=torch.int32, device=dev))
            dtype = self.src_k[0].dtype
            new_k, new_v = (torch.empty((s.layers, max(tokens), s.kv_heads, s.head_dim),
                                        dtype=dtype, device=dev) for _ in range(2))
            fill_pool([new_k, new_v], s.dtype, 12345)
            out = torch.empty((s.n_arrays, max(contexts), s.kv_heads, s.head_dim), dtype=dtype,
                              device=dev)
            self._slots = (tokens, contexts, slots, tables, new_k, new_v, out)
        return self._slots

    def write_kv(self) -> None:
        """One launch per request writes its new K and V rows into every layer."""
        from iekv import _native

        tokens, _, slots, _, new_k, new_v, _ = self._slot_inputs()
        h = self.stream.cuda_stream
        bs, L = self.w.shape.block_size, self.w.shape.layers
        stride = new_k[0].numel() * new_k.element_size()
        for n, sl in zip(tokens, slots):
            _native.call("iekv_write_slots_layers", self.src.native.handle, 0, L, bs,
                         new_k.data_ptr(), new_v.data_ptr(), stride, sl.data_ptr(), n, h)

    def write_kv_per_layer(self) -> None:
        """One launch per request and layer, as the reference calls write_kv per layer."""
        from iekv import _native

        tokens, _, slots, _, new_k, new_v, _ = self._slot_inputs()
        h = self.stream.cuda_stream
        bs = self.w.shape.block_size
        for n, sl in zip(tokens, slots):
            for layer in range(self.w.shape.layers):
                _native.call("iekv_write_slots", self.src.native.handle, layer, bs,
                             new_k[layer].data_ptr(), new_v[layer].data_ptr(), sl.data_ptr(),
                             n, h)

    def gather_context(self) -> None:
        """One launch per request gathers its context from every K and V array."""
        from iekv import _native

        _, contexts, _, tables, _, _, out = self._slot_inputs()
        h = self.stream.cuda_stream
        bs, A = self.w.shape.block_size, self.w.shape.n_arrays
        for n, table in zip(contexts, tables):
            nbytes = A * n * out[0, 0].numel() * out.element_size()
            _native.call("iekv_gather_rows_arrays", self.dst.native.handle, 0, A, bs,
                         table.data_ptr(), n, out.data_ptr(), nbytes, h)

    def gather_per_array(self) -> None:
        """One launch per request and array, as the reference gathers each cache apart."""
        from iekv import _native

        _, contexts, _, tables, _, _, out = self._slot_inputs()
        h = self.stream.cuda_stream
        bs = self.w.shape.block_size
        nbytes = out[0].numel() * out.element_size()
        for n, table in zip(contexts, tables):
            for a in range(self.w.shape.n_arrays):
                _native.call("iekv_gather_rows", self.dst.native.handle, a, bs,
                             table.data_ptr(), n, out[a].data_ptr(), nbytes, h)

    def verify_write_kv(self) -> bool:
        """Every request's slots hold its new K and V rows, each layer its own."""
        torch = self.torch
        tokens, _, slots, _, new_k, new_v, _ = self._slot_inputs()
        L = self.w.shape.layers
        arrays = self.src_k + self.src_v
        for n, sl in zip(tokens, slots):
            for a, t in enumerate(arrays):
                want = (new_k[a] if a < L else new_v[a - L])[:n]
                if not torch.equal(t.index_select(0, sl).view(torch.uint8),
                                   want.view(torch.uint8)):
                    return False
        return True

    def verify_gather(self, packed: bool = True) -> bool:
        """The context buffer holds the last request's rows of every array: packed as
        [2L, context] by the one-launch leg, one [context] slab per array otherwise."""
        torch = self.torch
        _, contexts, _, tables, _, _, out = self._slot_inputs()
        bs = self.w.shape.block_size
        n, table = contexts[-1], tables[-1].long()
        pos = torch.arange(n, device=table.device)
        rows_of = table[pos // bs] * bs + pos % bs
        flat = out.view(-1, *out.shape[2:])
        for a, cache in enumerate(self.dst_k + self.dst_v):
            got = flat[a * n:(a + 1) * n] if packed else out[a, :n]
            if not torch.equal(got.view(torch.uint8),
                               cache.index_select(0, rows_of).view(torch.uint8)):
                return False
        return True

    def direct(self) -> None:
        from iekv import _native

        hs = self._fork()
        for k, (s, d) in enumerate(zip(self.src_direct, self.dst_direct)):
            _native.call("iekv_copy_direct", self.src.native.handle, self.dst.native.handle,
                         s.data_ptr(), d.data_ptr(), s.numel(), hs[k % len(hs)])
        self._join()

    def direct_ids(self) -> None:
        """The direct leg with each request's table in host memory, as a serving loop
        holds it: iekv_copy_direct_ids checks the ids and carries them in the launch's
        kernel arguments (IEKV_INLINE_IDS per launch), so no kernel reads an id from
        device memory before its first data load."""
        from array import array

        from iekv import _native

        if not hasattr(self, "_host_tables"):
            self._host_tables = [(array("i", s.tolist()), array("i", d.tolist()))
                                 for s, d in zip(self.src_direct, self.dst_direct)]
        hs = self._fork()
        for k, (s, d) in enumerate(self._host_tables):
            _native.call("iekv_copy_direct_ids", self.src.native.handle, self.dst.native.handle,
                         s.buffer_info()[0], d.buffer_info()[0], len(s), hs[k % len(hs)])
        self._join()

    def _drop_in(self):
        """HipSlotCopier pair over the two pools (the drop-in Python API)."""
        if not hasattr(self, "_copiers"):
            from iekv.engine.copier import HipSlotCopier

            bs = self.w.shape.block_size
            self._copiers = (HipSlotCopier(self.src_k, self.src_v, bs),
                             HipSlotCopier(self.dst_k, self.dst_v, bs))
        return self._copiers

    def copier(self) -> None:
        """The drop-in Python path: HipSlotCopier.copy_blocks per request, given the
        request's block tables as Python lists (id checks and hand-over included),
        request k on request stream k mod S."""
        src, dst = self._drop_in()
        self._fork()
        S = len(self.streams)
        for k, (s, d) in enumerate(zip(self.w.src_tables, self.w.dst_tables)):
            dst.copy_blocks(src, s, d, stream=self.streams[k % S])
        self._join()

    def copier_pack_unpack(self) -> None:
        """The drop-in Python path of pack mode: read_blocks then write_blocks per request
        with the tables as Python lists (a new payload buffer per request, as the
        reference's KVTransfer holds one), request k on request stream k mod S."""
        src, dst = self._drop_in()
        self._fork()
        S = len(self.streams)
        for k, (s, d) in enumerate(zip(self.w.src_tables, self.w.dst_tables)):
            st = self.streams[k % S]
            dst.write_blocks(d, src.read_blocks(s, stream=st), stream=st)
        self._join()

    def pack_unpack(self) -> None:
        from iekv import _native

        hs = self._fork()
        for k, (s, d) in enumerate(zip(self.src_ids, self.dst_ids)):
            n, h, st = s.numel(), hs[k % len(hs)], self.stagings[k % len(hs)]
            _native.call("iekv_pack", self.src.native.handle, s.data_ptr(), n, st.data_ptr(),
                         st.numel(), h)
            _native.call("iekv_unpack", self.dst.native.handle, d.data_ptr(), n, st.data_ptr(),
                         st.numel(), h)
        self._join()

    def pack(self) -> None:
        """The pack half alone: every request gathered into its stream's staging buffer."""
        from iekv import _native

        hs = self._fork()
        for k, s in enumerate(self.src_ids):
            st = self.stagings[k % len(hs)]
            _native.call("iekv_pack", self.src.native.handle, s.data_ptr(), s.numel(),
                         st.data_ptr(), st.numel(), hs[k % len(hs)])
        self._join()

    def unpack(self) -> None:
        """The unpack half alone: each stream's staging buffer scattered onto its requests' ids."""
        from iekv import _native

        hs = self._fork()
        for k, d in enumerate(self.dst_ids):
            st = self.stagings[k % len(hs)]
            _native.call("iekv_unpack", self.dst.native.handle, d.data_ptr(), d.numel(),
                         st.data_ptr(), st.numel(), hs[k % len(hs)])
        self._join()

    def requests(self) -> None:
        """The direct leg's per-request launches issued by the library in one call
        (iekv_copy_direct_requests), request k on request stream k mod S."""
        import ctypes
        from array import array

        from iekv import _native

        if not hasattr(self, "_requests"):
            torch = self.torch
            self._requests = (array("i", [t.numel() for t in self.src_direct]),
                              torch.cat(self.src_direct), torch.cat(self.dst_direct))
        counts, src, dst = self._requests
        hs = self._fork()
        handles = (ctypes.c_void_p * len(hs))(*hs)
        _native.call("iekv_copy_direct_requests", self.src.native.handle, self.dst.native.handle,
                     len(counts), counts.buffer_info()[0], src.data_ptr(), dst.data_ptr(),
                     handles, len(hs), None)
        self._join()

    def _queue(self):
        """The request queue over the two pools and the step's tables as int32 arrays."""
        if not hasattr(self, "_handoff_queue"):
            import numpy as np

            from iekv.engine.queue import HandoffQueue

            self._handoff_queue = HandoffQueue(self.src, self.dst)
            tables = [(np.asarray(s, dtype=np.int32), np.asarray(d, dtype=np.int32))
                      for s, d in zip(self.w.src_tables, self.w.dst_tables)]
            self._queue_tables = tables
            self._queue_batch = (np.array([s.size for s, _ in tables], dtype=np.int32),
                                 np.concatenate([s for s, _ in tables]),
                                 np.concatenate([d for _, d in tables]))
        return self._handoff_queue

    def queue(self) -> None:
        """Every request submitted to the resident queue in one library call (its own
        descriptor and ticket each), then the last ticket waited for."""
        q = self._queue()
        q.submit_requests(*self._queue_batch)
        q.wait()

    def queue_py(self) -> None:
        """Every request submitted to the resident queue with its own Python call."""
        q = self._queue()
        for s, d in self._queue_tables:
            q.submit(s, d)
        q.wait()

    def queue_latency(self) -> list[float]:
        """Milliseconds from submitting each request alone to its completion."""
        q = self._queue()
        out = []
        for s, d in self._queue_tables:
            t0 = time.perf_counter()
            q.wait(q.submit(s, d))
            out.append(1000 * (time.perf_counter() - t0))
        return out

    def launch_latency(self) -> list[float]:
        """Milliseconds from issuing each request's direct launch (host ids, as
        iekv_copy_direct_ids takes them) to the host seeing it done (a stream
        synchronize): the per-launch path's counterpart of queue_latency."""
        from iekv import _native

        self._queue()
        out = []
        for s, d in self._queue_tables:
            t0 = time.perf_counter()
            _native.call("iekv_copy_direct_ids", self.src.native.handle, self.dst.native.handle,
                         s.ctypes.data, d.ctypes.data, s.size, self.stream.cuda_stream)
            self.stream.synchronize()
            out.append(1000 * (time.perf_counter() - t0))
        return out

    def stop_queue(self) -> None:
        if hasattr(self, "_handoff_queue"):
            self._handoff_queue.stop()

    def batched(self) -> None:
        from iekv import _native

        _native.call("iekv_copy_direct", self.src.native.handle, self.dst.native.handle,
                     self.src_all.data_ptr(), self.dst_all.data_ptr(), self.src_all.numel(),
                     self.stream.cuda_stream)

    def plain_copy(self) -> None:
        """A contiguous device-to-device copy of a known size (torch copy_), for reference."""
        torch = self.torch
        if not hasattr(self, "_plain"):
            # Random bytes, like the pools: on this GPU the bytes' values move the
            # rate a little (a contiguous copy of zeros ran 1.4% faster).
            n = 4 << 30
            device = self.src_k[0].device
            gen = torch.Generator(device=device)
            gen.manual_seed(7)
            self._plain = (torch.randint(0, 256, (n,), dtype=torch.uint8, device=device,
                                         generator=gen),
                           torch.zeros(n, dtype=torch.uint8, device=device))
        a, b = self._plain
        b.copy_(a)

    def host_roundtrip(self, steps: int, warmup: int) -> dict:
        """Offload every moved block to pinned host memory and restore it onto its dst id.

        One iekv_offload over the whole block list (the pack kernel writing the
        pinned image, 64 MiB of images per launch), then one iekv_restore (the
        unpack kernel reading it). Both are bounded by the host link, not HBM. Then, on a sample, the same calls once per block (the
        reference's pattern), and the drop-in tier path (_tier_roundtrip). The host
        image is pinned at exactly its size (iekv_host_alloc) and freed before the
        tier runs; the leg refuses to start when the host cannot hold what it pins
        (host_roundtrip_plan). Every phase logs a line as it starts.
        """
        from iekv import _native
        from iekv.engine.copier import HOST_STAGING_BYTES
        from iekv.engine.pools import pinned_empty, release_pinned

        torch = self.torch
        P = self.w.payload_bytes
        n = self.src_all.numel()
        k = min(n, 1024)
        plan = host_roundtrip_plan(self.w, k)
        check_host_budget(plan, host_memory_budget())

        def phase(msg: str) -> None:
            log(f"[bench] host_roundtrip: {msg}")

        phase(f"pinning {P / 1e9:.2f} GB (exactly the image; peak pinned "
              f"{plan['peak_pinned_bytes'] / 1e9:.2f} GB)")
        t0 = time.perf_counter()
        host = pinned_empty(P)
        pin_s = time.perf_counter() - t0
        staging = torch.empty(2 * HOST_STAGING_BYTES, dtype=torch.uint8,
                              device=self.src_k[0].device)
        side = torch.cuda.Stream(self.src_k[0].device)
        h = self.stream.cuda_stream

        def offload():
            _native.call("iekv_offload", self.src.native.handle, self.src_all.data_ptr(), n,
                         host.data_ptr(), P, staging.data_ptr(), staging.numel(), h,
                         side.cuda_stream)

        def restore():
            _native.call("iekv_restore", self.dst.native.handle, self.dst_all.data_ptr(), n,
                         host.data_ptr(), P, staging.data_ptr(), staging.numel(), h,
                         side.cuda_stream)

        phase(f"whole-list offload and restore, {warmup} warm-up and {steps} timed")
        for _ in range(warmup):
            offload()
            restore()
        torch.cuda.synchronize()
        d2h, h2d = [], []
        for _ in range(steps):
            a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            a.record(self.stream)
            offload()
            b.record(self.stream)     # the compute stream waits for the last copy
            restore()
            c.record(self.stream)     # after the last unpack
            torch.cuda.synchronize()
            d2h.append(a.elapsed_time(b))
            h2d.append(b.elapsed_time(c))
        # The same calls once per block, as the reference offloads one block per
        # eviction and restores one per tier hit (ie/core/block_manager.py:82,
        # 159-162), on a bounded sample of the blocks.
        bb = self.w.shape.block_bytes

        def offload_each():
            for i in range(k):
                _native.call("iekv_offload", self.src.native.handle,
                             self.src_all[i:].data_ptr(), 1, host.data_ptr() + i * bb, bb,
                             staging.data_ptr(), staging.numel(), h, side.cuda_stream)

        # As HipSlotCopier does, a pinned image is restored with the compute stream
        # as the copy stream (the unpack kernel reads it itself).
        def restore_each():
            for i in range(k):
                _native.call("iekv_restore", self.dst.native.handle,
                             self.dst_all[i:].data_ptr(), 1, host.data_ptr() + i * bb, bb,
                             staging.data_ptr(), staging.numel(), h, h)

        phase(f"one call per block on {k} blocks")
        offload_each()
        restore_each()
        torch.cuda.synchronize()
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record(self.stream)
        offload_each()
        b.record(self.stream)
        restore_each()
        c.record(self.stream)
        torch.cuda.synchronize()
        each_d2h, each_h2d = a.elapsed_time(b), b.elapsed_time(c)
        del host
        freed = release_pinned()
        phase(f"host image released ({freed / 1e9:.2f} GB)")
        tier = self._tier_roundtrip(k, phase)
        d2h_ms, h2d_ms = statistics.median(d2h), statistics.median(h2d)
        out = {"pinned_GB": round(P / 1e9, 2), "pin_alloc_s": round(pin_s, 2),
               "peak_pinned_GB": round(plan["peak_pinned_bytes"] / 1e9, 2),
               "d2h_ms": round(d2h_ms, 2), "h2d_ms": round(h2d_ms, 2),
               "d2h_GBps": round(P / (d2h_ms * 1e-3) / 1e9, 2),
               "h2d_GBps": round(P / (h2d_ms * 1e-3) / 1e9, 2),
               "roundtrip_ms": round(d2h_ms + h2d_ms, 2),
               "bound": "host link (PCIe Gen5 x16, 64 GB/s per direction theoretical)",
               "one_call_per_block": {
                   "blocks": k, "block_bytes": bb,
                   "d2h_GBps": round(k * bb / (each_d2h * 1e-3) / 1e9, 2),
                   "h2d_GBps": round(k * bb / (each_h2d * 1e-3) / 1e9, 2),
                   "d2h_us_per_block": round(1000 * each_d2h / k, 2),
                   "h2d_us_per_block": round(1000 * each_h2d / k, 2)},
               "through_the_tier": tier}
        log(f"[bench] host_roundtrip  {P / 1e9:.2f} GB pinned ({pin_s:.1f} s to pin): "
            f"D2H {out['d2h_GBps']} GB/s, H2D {out['h2d_GBps']} GB/s, "
            f"round trip {out['roundtrip_ms']} ms; one call per block ({k} blocks): "
            f"D2H {out['one_call_per_block']['d2h_GBps']} GB/s, "
            f"H2D {out['one_call_per_block']['h2d_GBps']} GB/s; through the tier "
            f"({tier['evictions_per_flush']} evictions per flush): D2H {tier['d2h_GBps']} GB/s, "
            f"H2D {tier['h2d_GBps']} GB/s")
        return out

    def _tier_roundtrip(self, k: int, phase, per_flush: int = 64) -> dict:
        """The same k blocks through the drop-in tier path, as the engine moves them.

        A host-payload HipSlotCopier queues ``per_flush`` evictions (read_block, the
        offload hook's call) and flushes them together, each block into a pinned
        buffer of its own (iekv_offload_blocks); the payloads are then restored as
        scattered tier entries (write_blocks -> iekv_restore_blocks), ``per_flush``
        per call. Times are wall-clock to completion, host work included.
        """
        from iekv.engine.copier import HipSlotCopier
        from iekv.engine.pools import release_pinned

        torch = self.torch
        bs, bb = self.w.shape.block_size, self.w.shape.block_bytes
        src = HipSlotCopier(self.src_k, self.src_v, bs, payload_location="host")
        dst = HipSlotCopier(self.dst_k, self.dst_v, bs)
        src_ids = [int(b) for b in self.src_all[:k].tolist()]
        dst_ids = [int(b) for b in self.dst_all[:k].tolist()]

        def offload():
            payloads = []
            for g in range(0, k, per_flush):
                payloads += [src.read_block(b) for b in src_ids[g:g + per_flush]]
                src.flush()
            return payloads

        def restore(payloads):
            for g in range(0, k, per_flush):
                dst.write_blocks(dst_ids[g:g + per_flush], payloads[g:g + per_flush])

        phase(f"tier warm-up: {k} evictions, {per_flush} per flush, then their restores")
        restore(offload())                      # warm-up: pinned buffers, kernels
        torch.cuda.synchronize()
        phase("tier offload (timed)")
        t0 = time.perf_counter()
        payloads = offload()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        phase("tier restore (timed)")
        restore(payloads)
        t3 = time.perf_counter()
        torch.cuda.synchronize()
        t4 = time.perf_counter()
        del payloads
        freed = release_pinned()
        phase(f"tier buffers released ({freed / 1e9:.2f} GB)")
        return {"blocks": k, "block_bytes": bb, "evictions_per_flush": per_flush,
                "d2h_GBps": round(k * bb / (t2 - t0) / 1e9, 2),
                "h2d_GBps": round(k * bb / (t4 - t2) / 1e9, 2),
                "host_us_per_block_offload": round(1e6 * (t1 - t0) / k, 2),
                "host_us_per_block_restore": round(1e6 * (t3 - t2) / k, 2)}

    def verify(self) -> bool:
        """Every destination tile equals its source tile (whole workload, on the GPU)."""
        torch = self.torch
        T = self.w.shape.tile_bytes
        ok = True
        for s_arr, d_arr in zip(self.src_k + self.src_v, self.dst_k + self.dst_v):
            s_tiles = s_arr.view(torch.uint8).view(-1, T)
            d_tiles = d_arr.view(torch.uint8).view(-1, T)
            for lo in range(0, self.src_all.numel(), 8192):
                si = self.src_all[lo:lo + 8192].long()
                di = self.dst_all[lo:lo + 8192].long()
                if not torch.equal(s_tiles.index_select(0, si), d_tiles.index_select(0, di)):
                    ok = False
        return ok

    def _tiles(self, arrays):
        T = self.w.shape.tile_bytes
        return [t.view(self.torch.uint8).view(-1, T) for t in arrays]

    def verify_pack(self) -> bool:
        """Each stream's staging buffer holds the block images, [n, 2L, T], of the last
        request packed on that stream."""
        torch = self.torch
        s = self.w.shape
        src_tiles = self._tiles(self.src_k + self.src_v)
        S = self.last_streams
        for k in range(max(0, len(self.src_ids) - S), len(self.src_ids)):
            ids = self.src_ids[k].long()
            n = ids.numel()
            image = self.stagings[k % S][:n * s.block_bytes].view(n, s.n_arrays, s.tile_bytes)
            if not all(torch.equal(image[:, a], tiles.index_select(0, ids))
                       for a, tiles in enumerate(src_tiles)):
                return False
        return True

    def verify_unpack(self) -> bool:
        """Every request's destination tiles equal the staging images it was unpacked from."""
        torch = self.torch
        s = self.w.shape
        dst_tiles = self._tiles(self.dst_k + self.dst_v)
        for k, d in enumerate(self.dst_ids):
            n = d.numel()
            staging = self.stagings[k % self.last_streams]
            image = staging[:n * s.block_bytes].view(n, s.n_arrays, s.tile_bytes)
            for a, tiles in enumerate(dst_tiles):
                if not torch.equal(image[:, a], tiles.index_select(0, d.long())):
                    return False
        return True

    def clear_dst(self) -> None:
        for t in self.dst_k + self.dst_v:
            t.zero_()

    def check(self, name: str) -> bool:
        """The check that fits what leg ``name`` leaves behind, right after it ran."""
        return {"pack": self.verify_pack, "unpack": self.verify_unpack,
                "write_kv": self.verify_write_kv,
                "write_kv_per_layer": self.verify_write_kv,
                "gather_context": self.verify_gather,
                "gather_per_array": lambda: self.verify_gather(packed=False)
                }.get(name, self.verify)()


def time_leg(legs: Legs, name: str, steps: int, warmup: int, per_launch: bool = True):
    """Warm up, then time ``steps`` steps twice.

    Pass 1 (the headline): HIP events only at step boundaries on the launch
    stream, so nothing is added between the launches of a step (the per-step
    times are kept in ``legs.step_ms``, and the host's time to issue each step in
    ``legs.issue_ms``). Pass 2 (when
    ``per_launch``): the same steps again with every kv_move launch timed by the
    library (iekv_profile_start/stop; the events ride in each launch's own
    dispatch packet). Returns (ms per step, wall seconds of pass 1,
    [(launch ms, algorithmic bytes, request)] from pass 2).
    """
    from iekv import _native

    torch = legs.torch
    step = getattr(legs, name)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    issue = []
    t0 = time.perf_counter()
    marks[0].record(legs.stream)
    for i in range(steps):
        h0 = time.perf_counter()
        step()
        marks[i + 1].record(legs.stream)
        issue.append(1000 * (time.perf_counter() - h0))
    torch.cuda.synchronize()
    legs.issue_ms[name] = issue
    wall = time.perf_counter() - t0
    ms_step = marks[0].elapsed_time(marks[-1]) / steps
    legs.step_ms[name] = [a.elapsed_time(b) for a, b in zip(marks, marks[1:])]
    legs.last_streams = len(legs.streams)
    plan = legs.plan(name)
    if not (per_launch and plan):
        return ms_step, wall, []
    # Pass 2 issues one launch at a time on the launch stream: launches on several
    # request streams run concurrently, and a launch's duration would then include
    # the time it shares the GPU with another.
    streams, stagings = legs.streams, legs.stagings
    legs.streams, legs.stagings = streams[:1], stagings[:1]
    try:
        # one spare slot: a leg that launches more than its plan says is caught below
        with _native.LaunchTimer(steps * len(plan) + 1) as timer:
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
        legs.last_streams = 1
    finally:
        legs.streams, legs.stagings = streams, stagings
    if len(timer.durations_ms) != steps * len(plan):
        raise RuntimeError(f"{name}: {len(timer.durations_ms)} launches timed, the leg's plan "
                           f"has {steps * len(plan)}")
    launches = [(ms, nbytes, r) for ms, (nbytes, r) in zip(timer.durations_ms, plan * steps)]
    return ms_step, wall, launches


def time_queue_leg(legs: Legs, name: str, steps: int, warmup: int):
    """Warm up, then time ``steps`` steps of a queue leg by the host clock: each step
    from its first submission to the completion of its last request (the queue's
    kernel stays resident over the whole pass, and a step ends only when the host
    has seen every request done). Then every request once more, each submitted and
    waited for alone (``legs.queue_ms``), and the queue stopped. Returns (ms per
    step, wall seconds, [])."""
    step = getattr(legs, name)
    legs.torch.cuda.synchronize()
    legs.launch_latency()                      # warm-up of the per-launch path
    legs.launch_ms = legs.launch_latency()     # before the queue's kernel starts
    for _ in range(warmup):
        step()
    times = []
    t0 = time.perf_counter()
    for _ in range(steps):
        h0 = time.perf_counter()
        step()
        times.append(1000 * (time.perf_counter() - h0))
    wall = time.perf_counter() - t0
    legs.step_ms[name] = times
    legs.issue_ms[name] = times
    legs.queue_ms = legs.queue_latency()
    stats = legs._handoff_queue.stats()
    legs.stop_queue()
    log(f"[bench] {name}: {stats['descriptors']} descriptors in {stats['launches']} kernel "
        f"launch(es)")
    return sum(times) / steps, wall, []


def summarize(legs: Legs, name: str, ms_step: float, launches, bytes_per_step: int, steps: int):
    w = legs.w
    if not launches:   # not a kv_move leg: one "launch" per step, timed by the step events
        launches = [(ms_step, bytes_per_step, 0)] * steps
    durations = [ms for ms, _, _ in launches]
    total_ms = sum(durations)
    moved = sum(nbytes for _, nbytes, _ in launches)
    per_request: dict[int, float] = {}
    for ms, _, r in launches:
        per_request[r] = per_request.get(r, 0.0) + ms
    req_ms = sorted(v / steps for v in per_request.values())
    gbs = bytes_per_step / (ms_step * 1e-3) / 1e9
    kernel_gbs = moved / (total_ms * 1e-3) / 1e9 if total_ms else 0.0
    out = {
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(statistics.median(legs.step_ms.get(name, [ms_step])), 4),
        # The host's time to issue one step's launches: the fastest timed step (a
        # full launch queue can only make the host wait longer). Close to
        # ms_per_step means the leg is bound by issuing launches, not by HBM.
        "host_issue_ms_per_step": round(min(legs.issue_ms.get(name, [0.0])), 4),
        "GBps": round(gbs, 1),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "kernel_GBps": round(kernel_gbs, 1),
        "launches_per_step": len(launches) // steps,
        "avg_launch_us": round(1000 * total_ms / max(1, len(durations)), 2),
        "blocks_per_s": round(w.num_blocks / (ms_step * 1e-3), 1),
    }
    if name in QUEUE_LEGS:
        # each request submitted and waited for alone: its latency seen from the host
        req_ms = sorted(getattr(legs, "queue_ms", None) or [ms_step])
        launch = sorted(getattr(legs, "launch_ms", None) or [0.0])
        out["launch_latency_ms"] = {"p50": round(launch[len(launch) // 2], 4),
                                    "p99": round(launch[min(len(launch) - 1,
                                                            int(0.99 * len(launch)))], 4)}
    if name in ("direct", "direct_ids", "copier", "requests", "pack_unpack",
                "copier_pack_unpack", "pack", "unpack", *SLOT_LEGS, *QUEUE_LEGS):
        out["ms_per_request"] = {"mean": round(statistics.fmean(req_ms), 4),
                                 "p50": round(req_ms[len(req_ms) // 2], 4),
                                 "p99": round(req_ms[min(len(req_ms) - 1,
                                                         int(0.99 * len(req_ms)))], 4),
                                 "max": round(req_ms[-1], 4)}
    log(f"[bench] {name:11s} {ms_step:9.3f} ms/step  {gbs:8.1f} GB/s "
        f"({out['pct_hbm_peak']:.1f}% of peak)  kernel {kernel_gbs:8.1f} GB/s  "
        f"{out['avg_launch_us']:.1f} us/launch  host issue {out['host_issue_ms_per_step']:.3f} "
        f"ms/step")
    return out, kernel_gbs, 1000 * total_ms / max(1, len(durations)), moved / max(1, len(durations))


def cpu_baseline(workload, budget_blocks: int, seed: int, min_seconds: float,
                 source_arrays) -> dict:
    """The reference handoff restated in NumPy (oracle/), single-threaded, on a bounded sample.

    The sample is the workload's first requests up to ``budget_blocks`` blocks, on
    host pools just large enough for them, with random src/dst ids; the handoff
    of the sample is repeated until ``min_seconds`` have passed. The host source
    pool holds the GPU leg's own source bytes (the first blocks of each of
    ``source_arrays``, N(0,1) values), and afterwards every moved destination
    tile is compared byte for byte with its source tile.
    """
    import numpy as np
    import torch

    from oracle.copier import LayeredSlotCopier, pack, unpack

    s = workload.shape
    sizes, total = [], 0
    for t in workload.src_tables:
        if total + len(t) > budget_blocks and sizes:
            break
        sizes.append(len(t))
        total += len(t)
    pool = min(total + 64, workload.src_pool_blocks)
    rng = np.random.default_rng(seed)
    src_ids = rng.permutation(pool)[:total]
    dst_ids = rng.permutation(pool)[:total]
    raw_view = {1: torch.uint8, 2: torch.int16, 4: torch.float32}[s.elem_bytes]
    rows = pool * s.block_size
    t0 = time.perf_counter()
    # The copies to host memory write every page once, so the timed copies do not pay
    # first-touch faults on the source; the destination pools are written here too.
    src_arrays = [a[:rows].view(raw_view).cpu().numpy() for a in source_arrays]
    src_k, src_v = src_arrays[:s.layers], src_arrays[s.layers:]
    dst_k = [np.zeros_like(a) for a in src_k]
    dst_v = [np.zeros_like(a) for a in src_v]
    log(f"[bench] cpu baseline: host pools of {pool} blocks (the GPU source's bytes) ready in "
        f"{time.perf_counter() - t0:.1f} s; {len(sizes)} requests, {total} blocks per pass")
    src = LayeredSlotCopier(src_k, src_v, s.block_size)
    dst = LayeredSlotCopier(dst_k, dst_v, s.block_size)
    passes = 0
    t0 = time.perf_counter()
    while True:
        at = 0
        for n in sizes:
            payloads = pack(src, src_ids[at:at + n])           # disaggregated.py:50
            unpack(dst, dst_ids[at:at + n], payloads)           # disaggregated.py:81-82
            at += n
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= min_seconds:
            break
    payload = total * s.block_bytes
    # Every moved tile, byte for byte: destination tile dst_ids[i] of each array
    # equals source tile src_ids[i] of the same array.
    ok = all(np.array_equal(d.reshape(pool, -1)[dst_ids], a.reshape(pool, -1)[src_ids])
             for d, a in zip(dst_k + dst_v, src_k + src_v))
    gbs = 2 * payload * passes / elapsed / 1e9
    log(f"[bench] cpu baseline: {passes} passes, {2 * payload * passes / 1e9:.2f} GB in "
        f"{elapsed:.2f} s = {gbs:.3f} GB/s")
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "seconds": round(elapsed, 2), "passes": passes, "checked": bool(ok),
            "ms_per_request": round(1000 * elapsed / (passes * len(sizes)), 3),
            "blocks_per_s": round(total * passes / elapsed, 1),
            "checked_what": (f"every moved tile ({total} blocks x {s.n_arrays} arrays) "
                             "equals its source tile byte for byte"),
            "sample": (f"{workload.name} shape, first {len(sizes)} requests ({total} blocks, "
                       f"{payload / 1e9:.2f} GB payload) on {pool}-block host pools holding "
                       f"the GPU source pool's N(0,1) bytes, random src/dst ids, repeated "
                       f"{passes}x; NumPy restatement of copier.py:18-31 driven as "
                       f"disaggregated.py:50,81-82; 1 of {os.cpu_count()} host cores")}


def _quantiles(ms: list[float]) -> dict:
    """Median, 10th and 90th percentile of launch durations, in microseconds."""
    us = sorted(1000 * x for x in ms)
    return {"p50_us": round(us[len(us) // 2], 3), "p10_us": round(us[len(us) // 10], 3),
            "p90_us": round(us[min(len(us) - 1, 9 * len(us) // 10)], 3), "launches": len(us)}


def launch_floor(device, configs=("cfg1", "cfg2"), seed: int = 0, reps: int = 400) -> dict:
    """What a launch costs before it moves a byte, and where a small request's time goes.

    In-dispatch durations (iekv_profile_start: events in each launch's own packet),
    launches issued one after another on one stream:
      * noop: iekv_noop, an empty kernel of 1 to 2,048 workgroups;
      * one_tile: iekv_copy_direct of one block between two one-array pools, tiles of
        4 to 64 KiB, ids in device memory, and iekv_copy_direct_ids (ids in the
        kernel arguments) for the same move;
      * requests: each request of the workloads' direct leg alone, with device ids and
        with host ids in the kernel arguments, against the bytes' time at peak.
    Host cost of issuing one launch: iekv_noop issuing many launches from C in one
    call, and a Python loop of one-launch calls.
    """
    import ctypes
    from array import array

    import torch

    from iekv import _native, workloads

    stream = torch.cuda.current_stream(device)
    h = stream.cuda_stream
    out: dict = {"unit": "microseconds", "noop": {}, "one_tile": {}, "host_us_per_launch": {},
                 "requests": {}, "hip_force_dev_kernarg": os.environ.get("HIP_FORCE_DEV_KERNARG")}

    def timed(issue, launches: int) -> list[float]:
        torch.cuda.synchronize()
        with _native.LaunchTimer(launches) as timer:
            issue()
            torch.cuda.synchronize()
        if len(timer.durations_ms) != launches:
            raise RuntimeError(f"{len(timer.durations_ms)} launches timed, {launches} issued")
        return timer.durations_ms

    for wg in (1, 8, 256, 2048):
        _native.call("iekv_noop", wg, 20, h)
        out["noop"][str(wg)] = _quantiles(timed(lambda: _native.call("iekv_noop", wg, reps, h),
                                                reps))
    log(f"[floor] noop: " + json.dumps(out["noop"]))

    n_host = 4000
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _native.call("iekv_noop", 1, n_host, h)
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    out["host_us_per_launch"]["noop_from_c"] = round(1e6 * (t1 - t0) / n_host, 3)
    noop = _native.lib().iekv_noop
    t0 = time.perf_counter()
    for _ in range(n_host):
        noop(1, 1, h)
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    out["host_us_per_launch"]["noop_python_loop"] = round(1e6 * (t1 - t0) / n_host, 3)

    # Back-to-back throughput: many empty launches issued together, no per-launch
    # events, spread over 1, 2 or 4 streams (each at the default priority); the
    # time per launch is what a stream of independent small requests pays.
    streams = [stream] + [torch.cuda.Stream(device) for _ in range(3)]
    out["noop_throughput_us_per_launch"] = {}
    for n_streams in (1, 2, 4):
        use = streams[:n_streams]
        per = 1000
        for _ in range(2):
            fork = torch.cuda.Event()
            fork.record(stream)
            for st in use[1:]:
                st.wait_event(fork)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for k in range(per):
                noop(1, 1, use[k % n_streams].cuda_stream)
            for st in use[1:]:
                done = torch.cuda.Event()
                done.record(st)
                stream.wait_event(done)
            b.record(stream)
            torch.cuda.synchronize()
        out["noop_throughput_us_per_launch"][str(n_streams)] = round(
            1000 * a.elapsed_time(b) / per, 3)
    log(f"[floor] host: " + json.dumps(out["host_us_per_launch"]) + "  throughput: "
        + json.dumps(out["noop_throughput_us_per_launch"]))

    ok = True
    for tile in (4096, 8192, 32768, 65536):
        blocks = 64
        src = torch.randint(0, 256, (blocks * tile,), dtype=torch.uint8, device=device)
        dst = torch.zeros(blocks * tile, dtype=torch.uint8, device=device)
        sp = _native.Pool([src.data_ptr()], tile, blocks, device.index or 0)
        dp = _native.Pool([dst.data_ptr()], tile, blocks, device.index or 0)
        sid = torch.tensor([5], dtype=torch.int32, device=device)
        did = torch.tensor([9], dtype=torch.int32, device=device)
        hs, hd = array("i", [5]), array("i", [9])

        def device_ids(n=reps):
            for _ in range(n):
                _native.call("iekv_copy_direct", sp.handle, dp.handle, sid.data_ptr(),
                             did.data_ptr(), 1, h)

        def host_ids(n=reps):
            for _ in range(n):
                _native.call("iekv_copy_direct_ids", sp.handle, dp.handle, hs.buffer_info()[0],
                             hd.buffer_info()[0], 1, h)

        device_ids(20)
        row = {"device_ids": _quantiles(timed(device_ids, reps)),
               "host_ids": _quantiles(timed(host_ids, reps))}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        device_ids(n_host // 4)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        row["host_us_per_call_python"] = round(1e6 * (t1 - t0) / (n_host // 4), 3)
        # The same one-block moves issued from C: iekv_copy_direct_requests with one
        # request per move on one stream (the library's own cost per launch).
        n_req = n_host // 4
        counts = array("i", [1] * n_req)
        many_s = sid.repeat(n_req)
        many_d = did.repeat(n_req)
        handles = (ctypes.c_void_p * 1)(h)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _native.call("iekv_copy_direct_requests", sp.handle, dp.handle, n_req,
                     counts.buffer_info()[0], many_s.data_ptr(), many_d.data_ptr(), handles, 1,
                     None)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        row["host_us_per_launch_c"] = round(1e6 * (t1 - t0) / n_req, 3)
        ok = ok and torch.equal(dst[9 * tile:10 * tile], src[5 * tile:6 * tile])
        out["one_tile"][str(tile)] = row
        sp.close()
        dp.close()
        del src, dst
    log(f"[floor] one tile: " + json.dumps(out["one_tile"]))

    for cfg in configs:
        w = workloads.make(cfg, seed, None)
        legs = Legs(w, device, seed, "paired", streams=1)
        bb = w.shape.block_bytes
        row = {"blocks_per_request": statistics.median(len(t) for t in w.src_tables),
               "bytes_per_request_median": int(2 * bb * statistics.median(
                   len(t) for t in w.src_tables))}
        for leg in ("direct", "direct_ids"):
            legs.clear_dst()
            _, _, launches = time_leg(legs, leg, 10, 3)
            row[leg] = _quantiles([ms for ms, _, _ in launches])
            ok = ok and legs.verify()
        row["bytes_at_peak_us"] = round(row["bytes_per_request_median"] / HBM_PEAK_GBS / 1e3, 3)
        out["requests"][cfg] = row
        log(f"[floor] {cfg}: " + json.dumps(row))
        del legs
        torch.cuda.empty_cache()
    out["verified"] = bool(ok)
    return out


def sweep(legs: Legs, names: list[str]) -> list[dict]:
    """Time each leg under the launch shapes iekv_set_launch offers (3 steps after 1 warm-up).

    Every workgroup order x chunk size (whole tiles, then 16 KiB down to 1 KiB
    chunks) at one block per workgroup, unroll 8, non-temporal; then the whole-tile
    runs of several blocks and the ordinary (temporal) accesses at each order's
    best chunk. ``order`` sets both workgroup orders (pool-writing and
    staging-writing launches).
    """
    from iekv import _native

    before = _native.get_launch()
    P = legs.w.payload_bytes
    rows = []

    def measure(run, unroll, nt, order, chunk):
        _native.set_launch(run, unroll, nt, order, order, chunk)
        row = {"run_blocks": run, "unroll": unroll, "nontemporal": nt, "order": order,
               "chunk_bytes": chunk}
        for name in names:
            ms, _, _ = time_leg(legs, name, 3, 1, per_launch=False)
            nbytes = 4 * P if name == "pack_unpack" else 2 * P
            row[name] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        rows.append(row)
        log("[sweep] " + json.dumps(row))

    try:
        for order in (0, 1, 2, 4, 5, 6):
            for chunk in (0, 16384, 8192, 4096, 2048, 1024):
                measure(1, 8, 1, order, chunk)
        for order in (0, 1, 2, 4, 5, 6):
            for run in (2, 4, 16):
                measure(run, 8, 1, order, 0)
            for unroll in (4, 16):
                measure(1, unroll, 1, order, 0)
            measure(1, 8, 0, order, 0)
            measure(1, 8, 0, order, 4096)
    finally:
        _native.set_launch(**before)
    for name in names:
        best = max(rows, key=lambda r: r[name])
        log(f"[sweep] best {name}: {best[name]} GB/s at " + json.dumps(
            {k: best[k] for k in ("run_blocks", "unroll", "nontemporal", "order",
                                  "chunk_bytes")}))
    return rows


def _chunk_ok(v: int) -> bool:
    return v == 0 or (64 <= v <= 1 << 20 and v & (v - 1) == 0)


# --ab keys that set one launch setting (iekv_set_launch / iekv_set_direct_chunk):
# the setting's name there and the values iekv.h allows.
LAUNCH_AB = {
    "direct_chunk": ("direct_chunk_bytes", _chunk_ok),
    "chunk": ("chunk_bytes", _chunk_ok),
    "order": ("order", lambda v: 0 <= v <= 7),
    "pack_order": ("pack_order", lambda v: 0 <= v <= 7),
    "unroll": ("unroll", lambda v: v in (1, 2, 4, 8, 16)),
    "nontemporal": ("nontemporal", lambda v: v in (0, 1)),
    "run": ("run_blocks", lambda v: 0 <= v <= 64),
}


def ab_ok(spec: str, config: str) -> bool:
    """Whether an --ab setting is well formed for this workload."""
    key, _, raw = spec.partition("=")
    values = [v for v in raw.split(",") if v]
    if not values:
        return False
    if key == "streams":
        return all(v.isdigit() and 1 <= int(v) <= 8 for v in values)
    if key == "slack":
        return config in ("cfg3", "cfg4") and all(v == "engine" or v.isdigit() for v in values)
    if key == "pad":
        return all(v.isdigit() and int(v) <= 4096 for v in values)
    if key in LAUNCH_AB:
        return all(v.isdigit() and LAUNCH_AB[key][1](int(v)) for v in values)
    return False


def ab(args, names: list[str], device) -> int:
    """In-process A/B of one setting, values alternated over rounds on one box.

    ``streams=1,2,4``: one set of pools, request streams switched between
    values. ``slack=64,6600,engine``: pools re-made for each value (cfg3 or
    cfg4 sized to the workload plus that many spare blocks, ``engine`` for the
    default pools), so every round also draws a new physical placement;
    ``pad=0,1``: the same, with that many unused blocks after each array. For
    these two the values run in reverse order every other round.
    ``direct_chunk=4096,8192,0`` (or another launch setting: ``chunk``,
    ``order``, ``pack_order``, ``unroll``, ``nontemporal``, ``run``): pools
    re-made for each round, and every value of the setting measured on the same
    pools within the round, so each placement compares all values. Prints one JSON line with every
    measurement and the per-value means.
    """
    import torch

    from iekv import _native, workloads

    key, _, raw = args.ab.partition("=")
    values = [v for v in raw.split(",") if v]
    legs_names = [n for n in names if n in HANDOFF_LEGS or n in SLOT_LEGS]
    rows, ok = [], True
    legs = None

    def measure(legs, rnd, value):
        """Time every leg on these pools, each checked right after its own run."""
        nonlocal ok
        w = legs.w
        row = {"round": rnd, "value": value,
               "pools": [w.src_pool_blocks, w.dst_pool_blocks]}
        for name in legs_names:
            if name not in ("gather_context", "gather_per_array"):
                legs.clear_dst()
            ms, _, _ = time_leg(legs, name, args.steps, args.warmup, per_launch=False)
            row[name] = round(sum(b for b, _ in legs.plan(name)) / (ms * 1e-3) / 1e9, 1)
            if not legs.check(name):
                row.setdefault("failed", []).append(name)
                ok = False
        rows.append(row)
        log("[ab] " + json.dumps(row))

    if key == "streams":
        counts = [int(v) for v in values]
        w = workloads.make(args.config, args.seed, args.slack, tp=args.tp)
        legs = Legs(w, device, args.seed, "separate" if args.separate_pools else "paired",
                    streams=max(counts), pad_blocks=args.pad)
        streams, stagings = legs.streams, legs.stagings
        for rnd in range(args.rounds):
            for n in counts:
                legs.streams, legs.stagings = streams[:n], stagings[:n]
                measure(legs, rnd, n)
        legs.streams, legs.stagings = streams, stagings
    elif key in LAUNCH_AB:
        before = _native.get_launch()
        try:
            for rnd in range(args.rounds):
                w = workloads.make(args.config, args.seed, args.slack, tp=args.tp)
                legs = Legs(w, device, args.seed,
                            "separate" if args.separate_pools else "paired",
                            streams=args.streams, pad_blocks=args.pad)
                for v in values:
                    _native.set_launch(**{LAUNCH_AB[key][0]: int(v)})
                    measure(legs, rnd, v)
                del legs
                torch.cuda.empty_cache()
        finally:
            _native.set_launch(**before)
    elif key == "pad":
        w = workloads.make(args.config, args.seed, args.slack, tp=args.tp)
        for rnd in range(args.rounds):
            # Re-made pools land on physical placements that repeat every few
            # allocations, one of them slow: reversing the order every other round
            # moves each value to other placements.
            for v in (values if rnd % 2 == 0 else values[::-1]):
                legs = Legs(w, device, args.seed,
                            "separate" if args.separate_pools else "paired",
                            streams=args.streams, pad_blocks=int(v))
                measure(legs, rnd, v)
                del legs
                torch.cuda.empty_cache()
    else:
        for rnd in range(args.rounds):
            for v in (values if rnd % 2 == 0 else values[::-1]):
                slack = None if v == "engine" else int(v)
                w = workloads.make(args.config, args.seed, slack, tp=args.tp)
                legs = Legs(w, device, args.seed,
                            "separate" if args.separate_pools else "paired",
                            streams=args.streams, pad_blocks=args.pad)
                measure(legs, rnd, v)
                del legs
                torch.cuda.empty_cache()
    means = {}
    for v in values:
        vv = int(v) if key == "streams" else v
        mine = [r for r in rows if r["value"] == vv]
        means[v] = {n: round(statistics.fmean(r[n] for r in mine), 1) for n in legs_names}
    print(json.dumps({"ab": key, "workload": args.config, "tp_share": args.tp,
                      "values": values, "rounds": args.rounds, "legs": legs_names, "unit": "GB/s",
                      "rows": rows, "mean": means, "verified": ok}))
    return 0 if ok else 1


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg3", help="cfg1..cfg5 (headline: cfg3)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--slack", type=int, default=None,
                    help="size cfg3's or cfg4's pools to the workload's needs plus SLACK blocks "
                         "(default: cfg3 64; cfg4 the cfg3 engine's pools, 49,598 blocks)")
    ap.add_argument("--legs", default="direct,pack_unpack,plain_copy",
                    help="comma list of direct, pack_unpack, pack, unpack, batched, copier, "
                         "copier_pack_unpack, requests, queue, queue_py, write_kv, "
                         "write_kv_per_layer, gather_context, gather_per_array, plain_copy, "
                         "host_roundtrip")
    ap.add_argument("--cpu-blocks", type=int, default=1536,
                    help="blocks in the CPU-baseline sample (0 skips it)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="minimum CPU-baseline time (the sample handoff repeats until then)")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--launch", default="",
                    help="run_blocks,unroll,nontemporal,order[,pack_order[,chunk_bytes"
                         "[,direct_chunk_bytes]]] for iekv_set_launch and "
                         "iekv_set_direct_chunk (default: the library's)")
    ap.add_argument("--sweep", action="store_true",
                    help="time the legs under every launch shape instead of the benchmark line")
    ap.add_argument("--tp", type=int, default=1,
                    help="measure one rank's share under head-sharded tensor parallelism "
                         "(H/tp KV heads per tile, same block tables)")
    ap.add_argument("--streams", type=int, default=0,
                    help="issue request k of the per-request legs on stream k mod STREAMS "
                         "(default 0: two streams when the workload's median request moves at "
                         "most 512 MiB each way, one otherwise; the per-launch timing pass "
                         "always uses one)")
    ap.add_argument("--ab", default="",
                    help="in-process A/B instead of the benchmark line: streams=1,2,4 (one set "
                         "of pools), slack=64,6600,engine (pools re-made per value; cfg3/cfg4), "
                         "pad=0,1 (pools re-made per value with that many unused blocks after "
                         "each array), or a launch setting such as direct_chunk=4096,8192,0 or "
                         "pack_order=0,4 (pools re-made per round, every value "
                         "on each)")
    ap.add_argument("--rounds", type=int, default=3, help="rounds of an --ab comparison")
    ap.add_argument("--floor", action="store_true",
                    help="measure the launch floor (empty kernels, one-tile moves, the small "
                         "workloads' requests) instead of the benchmark line")
    ap.add_argument("--pad", type=int, default=0,
                    help="unused blocks after each pool array (array stride = pool blocks + PAD)")
    ap.add_argument("--separate-pools", action="store_true",
                    help="allocate the two pools separately instead of as one reservation "
                         "(prefill pool first)")
    args = ap.parse_args()
    # A fatal signal prints every thread's Python stack before the process ends.
    faulthandler.enable()

    names = [x for x in args.legs.split(",") if x]
    if not args.sweep and not any(x in HANDOFF_LEGS for x in names):
        print(f"--legs needs one handoff leg ({', '.join(HANDOFF_LEGS)}) for the line's value",
              file=sys.stderr)
        return 2
    if args.ab and not ab_ok(args.ab, args.config):
        print("--ab takes streams=N,... (N in 1..8), a launch setting ("
              + ", ".join(f"{k}=V,..." for k in LAUNCH_AB)
              + "), pad=N,... (blocks after each pool array) or, for cfg3 and cfg4, "
              "slack=N|engine,...", file=sys.stderr)
        return 2
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the KV handoff runs on a single MI355X here "
              "(both pools in one HBM); multi-GPU runs are not part of this build.",
              file=sys.stderr)
        return 2

    if not 0 <= args.streams <= 8:
        print("--streams must be 0 (by request size) or 1..8", file=sys.stderr)
        return 2

    from iekv import workloads

    try:
        w = workloads.make(args.config, args.seed, args.slack, tp=args.tp)
    except ValueError as err:
        print(f"bench.py: {err}", file=sys.stderr)
        return 2

    import torch

    from iekv import _native

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda", 0)
    _native.lib()
    if args.launch:
        _native.set_launch(*[int(x) for x in args.launch.split(",")])
    if args.streams == 0:
        args.streams = request_streams(w)
    log(f"[bench] {w.name}: {w.num_requests} requests, {w.num_blocks} blocks, "
        f"P = {w.payload_bytes / 1e9:.2f} GB, tile {w.shape.tile_bytes} B, "
        f"{args.streams} request stream(s)")
    if args.ab:
        return ab(args, names, device)
    if args.floor:
        floor = launch_floor(device, seed=args.seed)
        print(json.dumps({"launch_floor": floor}), flush=True)
        return 0 if floor["verified"] else 1
    legs = Legs(w, device, args.seed, "separate" if args.separate_pools else "paired",
                streams=args.streams, pad_blocks=args.pad)
    P = w.payload_bytes
    if args.sweep:
        names = [x for x in args.legs.split(",")
                 if x in ("direct", "pack_unpack", "pack", "unpack", "batched")]
        rows = sweep(legs, names)
        ok = legs.verify()
        print(json.dumps({"sweep": w.name, "legs": names, "rows": rows, "verified": ok}))
        return 0 if ok else 1
    results: dict = {}
    verified: dict = {}
    primary = None
    for name in names:
        if name == "host_roundtrip":
            legs.clear_dst()
            results[name] = legs.host_roundtrip(max(1, min(args.steps, 3)), 1)
            if not args.no_verify:
                verified[name] = legs.verify()
                log(f"[bench] {name}: destination tiles equal source tiles: {verified[name]}")
            continue
        if name not in ("gather_context", "gather_per_array"):
            legs.clear_dst()
        if name in QUEUE_LEGS:
            ms, wall, launches = time_queue_leg(legs, name, args.steps, args.warmup)
        else:
            ms, wall, launches = time_leg(legs, name, args.steps, args.warmup)
        nbytes = 2 * (4 << 30) if name == "plain_copy" else sum(b for b, _ in legs.plan(name))
        res, kgbs, avg_us, avg_bytes = summarize(legs, name, ms, launches, nbytes, args.steps)
        res["wall_s"] = round(wall, 3)
        if name in ("pack_unpack", "copier_pack_unpack"):
            res["effective_handoff_GBps"] = round(2 * P / (ms * 1e-3) / 1e9, 1)
        if not args.no_verify and name != "plain_copy":
            verified[name] = legs.check(name)
            log(f"[bench] {name}: moved tiles equal their sources: {verified[name]}")
        results[name] = res
        if primary is None and name in HANDOFF_LEGS:
            primary = (name, ms, res, kgbs, avg_us, avg_bytes)

    cpu = None
    if args.cpu_blocks > 0:
        cpu = cpu_baseline(w, args.cpu_blocks, args.seed, args.cpu_seconds,
                           legs.src_k + legs.src_v)

    name, ms, res, kgbs, avg_us, avg_bytes = primary
    value = 2 * P / (ms * 1e-3) / 1e9
    launch = _native.get_launch()
    traffic, traffic_source = measured_traffic(w.name, args.tp, name, launch,
                                               args.separate_pools, avg_bytes)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_median": res["ms_per_step_median"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAMES[w.shape.dtype],
        "dtype_note": "the cache dtype; the kernels move its raw bits in 16-byte words",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.description}",
            "leg": name,
            "layers": w.shape.layers, "kv_heads": w.shape.kv_heads,
            "head_dim": w.shape.head_dim, "block_size": w.shape.block_size,
            "kv_dtype": w.shape.dtype, "requests": w.num_requests, "blocks": w.num_blocks,
            "payload_bytes": P, "tile_bytes": w.shape.tile_bytes, "tp_share": args.tp,
            "request_streams": args.streams,
            "launch": launch,
            "pools": ("two allocations" if args.separate_pools
                      else "one allocation, prefill pool first"),
        },
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "blocks_per_s": res["blocks_per_s"],
        "ms_per_request": res.get("ms_per_request"),
        "legs": results,
        "verified": verified,
        "roofline": {"bound": "hbm", "achieved": round(kgbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_source,
                     "kernel": "kv_queue" if name in QUEUE_LEGS else f"kv_move ({name})",
                     "avg_launch_us": round(avg_us, 2),
                     "algorithmic_bytes_per_launch": int(avg_bytes)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if all(verified.values()) else 1


if __name__ == "__main__":
    sys.exit(main())
