"""CPU oracle for the KV-cache handoff — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline). The product (``inference-engine_amd/iekv``) never imports it.

Modules:
  copier     NumPy restatement of LayeredSlotCopier (ie/engine/copier.py:6-38) and of
             the per-request handoff loops (ie/serve/disaggregated.py:50, 81-82).
  block_ids  Brute-force restatement of the free-list id assignment
             (ie/core/block_manager.py:50, 87-104, 178-198).

How each function is pinned (a function with no such check would be marked
"parity unpinned" here; none is):
  * tile addressing (`_span`, read_block, write_block): the reference's layout
    KATs (tests/test_paged_attention.py:54-70, gather slots [12,13,14,15,4,5]
    for table [3,1], bs 4; write slots [9,0,5]) re-run through this copier;
    closed form dst[a][d*T:(d+1)*T] == src[a][s*T:(s+1)*T] with untouched
    guard blocks; golden pool digests written by the reference itself
    (tests/golden/*.json);
  * bytes_moved: the reference's own counter values in the golden fixtures;
  * free-list ids: the reference's block-manager tests
    (tests/test_block_manager.py:25-83) and golden block tables recorded
    from the reference's engines.
"""
