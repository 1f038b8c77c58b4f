"""Expert dispatch and tile schedule in numpy (oracle; test infrastructure only).

dispatch() restates build_expert_dispatch (kernel.py:327-382): flat top-k slot
i = t*top_k + k is local when ids[i] - offset lies in [0, E_local) (kernel.py:271-272,
:313-314); token_counts is the histogram over local experts (kernel.py:357);
expert_start its exclusive cumulative sum with a leading 0 (kernel.py:358-360); each
local slot is placed in its expert's bucket with token = i // top_k (kernel.py:317) and
its routing weight. The reference claims bucket positions with atomics, so its order
inside a bucket is run-dependent (kernel.py:330-333); this oracle (and the HIP kernels)
use the stable order: ascending flat slot inside each bucket.

tile_schedule() restates build_tile_schedule (kernel.py:384-407), and work_items() the
HIP library's equivalent list of (expert, first row, rows) runs.
"""
from __future__ import annotations

import numpy as np


def dispatch(topk_ids: np.ndarray, topk_weights: np.ndarray, local_expert_offset: int,
             num_local_experts: int = 32):
    ids = np.asarray(topk_ids, dtype=np.int64)
    T, top_k = ids.shape
    flat = ids.reshape(-1) - int(local_expert_offset)
    local = (flat >= 0) & (flat < num_local_experts)
    slots = np.nonzero(local)[0]
    le = flat[slots]
    order = np.argsort(le, kind="stable")
    sorted_slot = slots[order].astype(np.int32)
    counts = np.bincount(le, minlength=num_local_experts).astype(np.int32)
    start = np.zeros(num_local_experts + 1, dtype=np.int32)
    start[1:] = np.cumsum(counts)
    return {
        "expert_count": counts,
        "expert_start": start,
        "sorted_slot": sorted_slot,
        "sorted_token": (sorted_slot // top_k).astype(np.int32),
        "sorted_weight": np.asarray(topk_weights, dtype=np.float32).reshape(-1)[sorted_slot],
        "token_nlocal": local.reshape(T, top_k).sum(axis=1).astype(np.int32),
        "local_mask": local.reshape(T, top_k),
    }


def tile_schedule(token_counts: np.ndarray, block_m: int):
    """(tile_expert_ids, tile_local_m, total_tiles): tile j of expert e covers bucket rows
    [m*block_m, (m+1)*block_m) of e, tiles ordered by expert (kernel.py:388-405)."""
    counts = np.asarray(token_counts, dtype=np.int64)
    tiles = (counts + block_m - 1) // block_m
    start_tile = np.zeros(len(counts) + 1, dtype=np.int64)
    start_tile[1:] = np.cumsum(tiles)
    total = int(start_tile[-1])
    idx = np.arange(total)
    tile_expert = np.searchsorted(start_tile[1:], idx, side="right").astype(np.int32)
    tile_local_m = (idx - start_tile[tile_expert]).astype(np.int32)
    return tile_expert, tile_local_m, total


def work_items(expert_count: np.ndarray, expert_start: np.ndarray, rows_per_item: int) -> np.ndarray:
    """[n, 4] int32 rows (expert, first sorted row, rows, first item of the expert |
    items of the expert << 16): each expert's bucket cut into runs of at most
    rows_per_item rows, experts in ascending order. Above 32 rows per item the runs are
    balanced: the run length is ceil(n / ceil(n / rows_per_item)) rounded up to 16."""
    out = []
    for e, n in enumerate(np.asarray(expert_count)):
        n = int(n)
        if n == 0:
            continue
        chunk = rows_per_item
        if rows_per_item > 32:
            nmax = -(-n // rows_per_item)
            chunk = min(rows_per_item, ((-(-n // nmax)) + 15) // 16 * 16)
        starts = list(range(0, n, chunk))
        first = len(out)
        for c in starts:
            out.append((e, int(expert_start[e]) + c, min(chunk, n - c), first | (len(starts) << 16)))
    return np.asarray(out, dtype=np.int32).reshape(-1, 4)
