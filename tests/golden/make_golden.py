"""Writes the committed golden fixtures from the CPU oracle (run on the CPU, once).

    python tests/golden/make_golden.py

config1_single_decode.npz   single-sequence 128-token decode on a random 8-block table:
                            inputs (raw fp16 bits) and the FP64 dense-attention output
config2_prompt_append.json  prompt append of 2048 tokens x 22 layers into a 4096-block pool
                            with 30% pre-occupied by 10 filler requests and a seeded free
                            list: the prompt's block table and slot mapping, and BLAKE2b
                            digests of the prompt K/V bytes and of the whole final pool
                            (NaN-poisoned before the appends)

The pool of config 2 is produced by the oracle's restatement of the reference allocator's
LIFO rules and chunked append; the GPU test replays the same steps through the product
allocator and must produce the same digest.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import paged_reference as ref  # noqa: E402
from tests import workloads  # noqa: E402


def digest(array: np.ndarray) -> str:
    return hashlib.blake2b(np.ascontiguousarray(array).view(np.uint8), digest_size=32).hexdigest()


def config1() -> None:
    w = workloads.single_decode()
    expected = ref.dense_attention_fp64(torch.from_numpy(w.query), torch.from_numpy(w.key), torch.from_numpy(w.value))
    np.savez(
        os.path.join(HERE, "config1_single_decode.npz"),
        query=w.query.view(np.uint16),
        key=w.key.view(np.uint16),
        value=w.value.view(np.uint16),
        table=np.asarray(w.table, dtype=np.int64),
        layer=np.int64(w.layer),
        num_blocks=np.int64(w.num_blocks),
        expected_fp64=expected.numpy(),
    )


def config2_pool(w: workloads.PromptAppend) -> tuple[np.ndarray, list]:
    """The oracle's pool after the filler appends and the prompt append."""
    pool = np.full((22, 2, w.num_blocks, 16, 4, 64), ref.NAN_F16_BITS, dtype=np.uint16)
    lifo = ref.LifoFreeList(list(w.free_order))
    for index, blocks in enumerate(w.filler_blocks):
        key, value = w.filler_kv(index)
        table = lifo.grow_to(f"filler{index}", key.shape[1])
        ref.reference_append(pool, table, 0, key.view(np.uint16), value.view(np.uint16))
    key, value = w.prompt_kv()
    table = lifo.grow_to("prompt", key.shape[1])
    ref.reference_append(pool, table, 0, key.view(np.uint16), value.view(np.uint16))
    return pool, table


def config2() -> None:
    w = workloads.prompt_append()
    pool, table = config2_pool(w)
    key, value = w.prompt_kv()
    slots = [table[p // 16] * 16 + p % 16 for p in range(w.prompt_tokens)]
    record = {
        "seed": w.seed,
        "num_blocks": w.num_blocks,
        "filler_blocks": w.filler_blocks,
        "prompt_table": [int(b) for b in table],
        "prompt_slot_mapping": [int(s) for s in slots],
        "prompt_key_blake2b": digest(key.view(np.uint16)),
        "prompt_value_blake2b": digest(value.view(np.uint16)),
        "pool_blake2b": digest(pool),
    }
    with open(os.path.join(HERE, "config2_prompt_append.json"), "w") as handle:
        json.dump(record, handle, indent=1)


if __name__ == "__main__":
    config1()
    config2()
    print("golden fixtures written to", HERE)
