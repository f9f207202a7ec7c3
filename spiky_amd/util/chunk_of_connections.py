"""ChunkOfConnections: the reference's connection-buffer format
(src/spiky/util/chunk_of_connections.py:15-46), produced and consumed here by
this library's own code.

Buffer layout (int32): groups of (4 + 2*single_group_size) ints,
  header (source_id, synapse_meta_index, n_targets, shift_to_next_group)
  body   (synapse_meta_index_i, target_id_i) x single_group_size
A list starts at a group whose source_id > 0; further groups of the list have
source_id == 0 and are reached through shift_to_next_group (in int32 units,
0 = end of list).  Pairs with target_id == 0 are padding.
"""
import numpy as np
import torch


class ChunkOfConnections(object):
    def __init__(self, connections: torch.Tensor, single_group_size: int, weights: torch.Tensor = None):
        self._connections = connections
        self._weights = weights
        self._single_group_size = single_group_size

    def get_connections(self):
        return self._connections

    def get_weights(self):
        return self._weights

    def get_single_group_size(self):
        return self._single_group_size

    def recycle(self):
        self._connections = None


def parse_connections(connections, single_group_size, ids_shift=0):
    """Returns (source_ids, target_ids) int64 arrays of every synapse in the
    buffer, ids_shift applied, in list order."""
    buf = connections.detach().cpu().numpy().astype(np.int64, copy=False) \
        if isinstance(connections, torch.Tensor) else np.asarray(connections, dtype=np.int64)
    g = 4 + 2 * int(single_group_size)
    n_groups = buf.size // g
    if n_groups == 0:
        return np.zeros(0, np.int64), np.zeros(0, np.int64)
    groups = buf[:n_groups * g].reshape(n_groups, g)
    heads = np.nonzero(groups[:, 0] > 0)[0]
    src_of_group = np.full(n_groups, -1, dtype=np.int64)
    for h in heads.tolist():
        cur = h
        steps = 0
        while True:
            src_of_group[cur] = groups[h, 0]
            shift = int(groups[cur, 3])
            if shift == 0:
                break
            if shift % g != 0:
                raise ValueError("malformed connections buffer: shift is not a whole group")
            cur += shift // g
            steps += 1
            if cur < 0 or cur >= n_groups or steps > n_groups:
                raise ValueError("malformed connections buffer: broken group list")
    used = src_of_group >= 0
    body = groups[used, 4:].reshape(-1, int(single_group_size), 2)
    tg = body[:, :, 1]
    src = np.repeat(src_of_group[used], int(single_group_size)).reshape(tg.shape)
    keep = tg > 0
    return src[keep] + ids_shift, tg[keep] + ids_shift


def build_connections(source_ids, offsets, targets, single_group_size, synapse_meta_index=0,
                      device=None):
    """CSR (source_ids[i] -> targets[offsets[i]:offsets[i+1]], ascending) ->
    ChunkOfConnections buffer in the format above."""
    sgs = int(single_group_size)
    g = 4 + 2 * sgs
    source_ids = np.asarray(source_ids, dtype=np.int64)
    offsets = np.asarray(offsets, dtype=np.int64)
    targets = np.asarray(targets, dtype=np.int64)
    counts = offsets[1:] - offsets[:-1]
    n_grp = np.maximum((counts + sgs - 1) // sgs, 0)
    total = int(n_grp.sum())
    out = np.zeros((max(total, 1), g), dtype=np.int32)
    row = 0
    for i in range(source_ids.size):
        c = int(counts[i])
        if c == 0:
            continue
        k = int(n_grp[i])
        tl = targets[offsets[i]:offsets[i + 1]]
        for j in range(k):
            r = out[row + j]
            r[0] = source_ids[i] if j == 0 else 0
            r[1] = synapse_meta_index
            r[2] = c if j == 0 else 0
            r[3] = g if j + 1 < k else 0
            part = tl[j * sgs:(j + 1) * sgs]
            r[4:4 + 2 * part.size:2] = synapse_meta_index
            r[5:5 + 2 * part.size:2] = part
        row += k
    t = torch.from_numpy(out[:total].reshape(-1) if total else np.zeros(g, dtype=np.int32))
    if device is not None:
        t = t.to(device)
    return ChunkOfConnections(t, sgs)


def create_identity_mapping(N: int, synapse_meta_index: int = 0, delta: int = 0, device=None):
    """Neuron i -> i + delta for i in [1, N], single_group_size = 1."""
    ids = np.arange(1, N + 1, dtype=np.int64)
    return build_connections(ids, np.arange(N + 1, dtype=np.int64), ids + delta, 1,
                             synapse_meta_index, device)


def repeat_connections_incrementing_source(chunk_of_connections: ChunkOfConnections, n_repeats: int):
    """Copies every list n_repeats times, the k-th copy with source id + k
    (reference chunk_of_connections.py:117-150)."""
    sgs = chunk_of_connections.get_single_group_size()
    src, tg = parse_connections(chunk_of_connections.get_connections(), sgs, 0)
    if src.size == 0:
        return ChunkOfConnections(chunk_of_connections.get_connections().clone(), sgs)
    order = np.lexsort((tg, src))
    src, tg = src[order], tg[order]
    uniq, start = np.unique(src, return_index=True)
    offs = np.append(start, src.size)
    new_src = (uniq[None, :] + np.arange(n_repeats)[:, None]).reshape(-1)
    lens = offs[1:] - offs[:-1]
    new_offs = np.zeros(new_src.size + 1, dtype=np.int64)
    new_offs[1:] = np.cumsum(np.tile(lens, n_repeats))
    new_tg = np.tile(tg, n_repeats)
    dev = chunk_of_connections.get_connections().device
    return build_connections(new_src, new_offs, new_tg, sgs, 0, dev)
