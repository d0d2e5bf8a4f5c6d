"""CPU oracle for the paged KV-cache hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference implementation's algorithm for the path
(PagedCore's src/pagedcore/attention.py and src/pagedcore/kv_cache.py) so that the GPU
product can be checked against it. Only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import it, and only as the checker or the timed CPU baseline; the
product package (pagedcore_amd) never imports, links or calls anything here.

Contents (each function cites the reference lines it restates):
  paged_reference.reference_paged_attention   attention.py:14-53 (default path, op for op)
  paged_reference.reference_append            kv_cache.py:161-172 (chunked copy order)
  paged_reference.reference_write_decode      kv_cache.py:242-245
  paged_reference.reference_assert_accounting kv_cache.py:314-357 (allocator invariants)
  paged_reference.LifoFreeList                kv_cache.py:86,158,197-201,297 (block choice)
  paged_reference.dense_attention_fp64        tests/unit/test_attention.py:173-179 (FP64 oracle)
  decoder_reference.*                         dense.py, decoder.py:70-100,202-240 (TinyLlama forward, generate)

How each one is pinned (tests/test_oracle.py): the reference tests' known answers (exact
3, exact 100*(h//8)+16, exact 0.25, tiny probabilities > 0, +-1000 scores) and FP64
agreement at 2e-3 pin reference_paged_attention; closed forms (q = 0 gives the mean of V,
a dominant key gives its value) and a pure-Python brute force pin dense_attention_fp64;
the reference tests' expected block tables ((0, 2, 3)/(1,), (2, 0, 3, 4), (0, 2), the
blocker relation) and the slot closed form pool[l, k, tbl[p // 16], p % 16] == src[l, p]
pin the append and the free list; the element closed form of the decode write at lengths
1..2048 pins reference_write_decode; the reference tests' counts (CapacityCounts(4, 0, 4,
4, 2, 34) after a staged step, the counts through create/append/release) and one planted
corruption per message (in the reference's check order) pin reference_assert_accounting.
Planted mistakes (wrong head mapping, missing 1/8 scale, transposed page, FIFO free list,
an off-by-one decode slot) are shown to fail those checks. The decoder oracle is pinned in
tests/test_oracle_decoder.py. No function is left parity-unpinned.
"""
