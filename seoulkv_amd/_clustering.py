"""Spherical hierarchical IVF over L2-normalised keys (host prefill, torch).

Restates the reference ``_clustering.py:18-236``: a coarse spherical k-means
(``coarse_iters`` Lloyd steps seeded by ``randperm``), leaves allocated to
coarse buckets in proportion to their occupancy, one batched local spherical
k-means per bucket, and finally each key's two best leaves as its two posting
lists (spill 2), emitted as CSR.

The clustering depends on torch's RNG stream and on the exact sequence of
floating-point operations, so the sequence of torch calls below is kept the
same as the reference's: the same generators and seeds, the same score-chunk
sizes and the same reductions.  Any change here changes which centroid a key
lands in.  Each block cites the reference lines it restates.

Two deliberate differences, both on a GPU build device only (the CPU build,
the one the golden vectors pin, is the reference's sequence):

* the leaf seeds of the batched local solves are drawn from a CPU generator
  on every build device and then moved (the reference draws them from a
  generator on the build device, ``_clustering.py:125,177``), so a GPU build
  starts from the same seeds as the CPU build;
* the centroid sums (the reference's ``index_add_`` / ``scatter_add_``,
  ``:27,192``) are accumulated in 64-bit fixed point (``fixed_row_sums``):
  on a GPU those float additions are atomics whose order varies from run to
  run, integer additions give the same bits in every order, so two GPU
  builds of the same keys are identical.  The sums are then exact to 2^-40
  per term, at least as accurate as the CPU's sequential FP32 sums.

The two indexes then differ only where floating-point rounding on the GPU
changes an assignment.
"""

from __future__ import annotations

import torch

EPS = 1e-12
SCORE_BUDGET = 16 * 2**20  # FP32 score elements per slab (64 MiB)
FIXED_ONE = 2.0**40  # fixed-point unit of the GPU centroid sums


def fixed_row_sums(out_rows: int, index: torch.Tensor, src: torch.Tensor, dim: int = 0):
    """Order-independent sums of the rows of ``src`` (|elements| <= 1, at
    most 2^20 rows per sum) into ``out_rows`` buckets along ``dim`` by
    ``index``: each element is rounded to a multiple of 2^-40 and summed as
    a 64-bit integer (|sum| <= 2^60), so every summation order gives the same
    result.  ``dim=0``: ``src`` [n, d], ``index`` [n] (``index_add_``);
    ``dim=1``: ``src`` [b, n, d], ``index`` [b, n] (``scatter_add_``)."""
    q = torch.round(src.double() * FIXED_ONE).long()
    if dim == 0:
        acc = torch.zeros(out_rows, src.shape[1], dtype=torch.long, device=src.device)
        acc.index_add_(0, index, q)
    else:
        acc = torch.zeros(src.shape[0], out_rows, src.shape[2], dtype=torch.long,
                          device=src.device)
        acc.scatter_add_(1, index[..., None].expand(-1, -1, src.shape[2]), q)
    return (acc.double() / FIXED_ONE).to(src.dtype)


def score_rows(n_centroids: int) -> int:
    # reference _clustering.py:9-10 (_score_rows)
    return max(1, min(8192, SCORE_BUDGET // n_centroids))


def withdraw(capacity: torch.Tensor, total: int) -> torch.Tensor:
    """Take ``total`` units from donors in order, each at most its capacity
    (reference ``_clustering.py:13-15``, ``_withdraw``)."""
    remaining = (total - capacity.cumsum(0)).clamp_min(0)
    return torch.cat((remaining.new_tensor([total]), remaining[:-1])) - remaining


def spherical_kmeans(x: torch.Tensor, k: int, iters: int, seed: int) -> torch.Tensor:
    """Lloyd iterations on the unit sphere (cosine assignment; reference
    ``_clustering.py:18-32``, ``_kmeans``)."""
    n = x.shape[0]
    gen = torch.Generator().manual_seed(seed)
    cent = x[torch.randperm(n, generator=gen)[:k].to(x.device)].clone()
    rows = score_rows(k)
    for _ in range(iters):
        label = torch.empty(n, dtype=torch.long, device=x.device)
        for start in range(0, n, rows):
            label[start : start + rows] = (x[start : start + rows] @ cent.t()).argmax(1)
        if x.device.type == "cpu":
            sums = torch.zeros_like(cent).index_add_(0, label, x)
        else:
            sums = fixed_row_sums(k, label, x)
        count = torch.bincount(label, minlength=k).unsqueeze(1).float()
        cent = torch.where(count > 0, sums / count.clamp_min(1), cent)
        cent = cent / cent.norm(dim=-1, keepdim=True).clamp_min(1e-9)
    return cent


def midrise(x: torch.Tensor, bits: int) -> torch.Tensor:
    """Max-abs mid-rise quantiser with 2**bits levels per row (reference
    ``_clustering.py:35-41``, ``_midrise``)."""
    a = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-9)
    levels = 2**bits
    step = 2 * a / levels
    return -a + (torch.clamp(torch.floor((x + a) / step), 0, levels - 1) + 0.5) * step


def allocate_leaves(counts: torch.Tensor, n_leaves: int) -> torch.Tensor:
    """Exactly ``n_leaves`` leaves over the coarse buckets, proportional to
    occupancy, at least one per non-empty bucket (largest remainders first;
    reference ``_clustering.py:44-70``, ``_allocate_leaves``)."""
    raw = counts.float() * (n_leaves / max(float(counts.sum()), 1.0))
    alloc = torch.floor(raw).long()
    alloc = torch.where(counts > 0, alloc.clamp_min(1), torch.zeros_like(alloc))
    delta = n_leaves - int(alloc.sum())
    if delta > 0:
        gain = raw - alloc.float()
        gain[counts == 0] = -torch.inf
        alloc[gain.topk(delta).indices] += 1
    elif delta < 0:
        removable = alloc > 1
        loss = raw - alloc.float()
        loss[~removable] = torch.inf
        if -delta <= int(removable.sum()):
            alloc[(-loss).topk(-delta).indices] -= 1
        else:
            # Several leaves may have to come back from one donor; never take
            # a bucket's last leaf.
            donors = loss.argsort(stable=True)
            alloc[donors] -= withdraw((alloc[donors] - 1).clamp_min(0), -delta)
    if int(alloc.sum()) != n_leaves:
        raise RuntimeError(
            f"hierarchical IVF leaf allocation {int(alloc.sum())} != {n_leaves}"
        )
    return alloc


def _solve_bucket_alone(x, size, nleaf, iters, seed):
    """A bucket too large to pad into a batch gets its own k-means
    (reference ``_clustering.py:149-153``)."""
    if size < nleaf:
        return x[torch.arange(nleaf, device=x.device) % size]
    return spherical_kmeans(x, nleaf, iters, seed)


def hierarchical_ivf(
    keys: torch.Tensor,
    n_leaves: int,
    spill: int,
    seed: int,
    coarse_clusters: int = 128,
    coarse_iters: int = 4,
    local_iters: int = 10,
    batch_coarse: int = 16,
):
    """Return ``(centroids, csr_values, csr_offsets, counts, labels, stats)``.

    ``keys`` are unit-norm fp32 rows.  ``labels[i]`` holds key i's ``spill``
    best leaves; the CSR lists every key under each of them, ordered by key.
    Reference ``_clustering.py:73-236`` (``_refined_hierarchical_ivf``).
    """
    n, d = keys.shape
    dev = keys.device
    # coarse k-means and assignment (reference :93-99)
    k0 = min(max(2, coarse_clusters), n_leaves, n)
    c0 = spherical_kmeans(keys, k0, coarse_iters, seed)
    coarse = torch.empty(n, dtype=torch.long, device=dev)
    for start in range(0, n, 8192):
        coarse[start : start + 8192] = (keys[start : start + 8192] @ c0.t()).argmax(1)

    # leaves per coarse bucket, topped up to `spill` per active bucket (:105-118)
    counts0 = torch.bincount(coarse, minlength=k0)
    leaves = allocate_leaves(counts0, n_leaves)
    active = counts0 > 0
    if bool((leaves[active] < spill).any()):
        # Every key needs ``spill`` distinct lists: move leaves from buckets
        # with spare leaves to under-provisioned ones, keeping the total.
        need = (spill - leaves).clamp_min(0) * active
        spare = (leaves - spill).clamp_min(0)
        deficit = int(need.sum())
        if int(spare.sum()) < deficit:
            raise ValueError("not enough fine leaves for distinct spill lists")
        donors = spare.argsort(descending=True, stable=True)
        leaves += need
        leaves[donors] -= withdraw(spare[donors], deficit)
    # bucket order and starts (:119-126); the seed generator is a CPU one on
    # every device (see the module note)
    leaf_start = leaves.cumsum(0) - leaves
    order = torch.argsort(coarse, stable=True)
    coarse_start = counts0.cumsum(0) - counts0
    cent = torch.empty(n_leaves, d, dtype=keys.dtype, device=dev)
    labels = torch.empty(n, spill, dtype=torch.long, device=dev)
    batch_coarse = max(1, int(batch_coarse))
    gen = torch.Generator().manual_seed(seed + 0x48494552)
    alone = 0

    for b0 in range(0, k0, batch_coarse):  # batches of coarse buckets (:128-217)
        b1 = min(b0 + batch_coarse, k0)
        cb = counts0[b0:b1]
        lb = leaves[b0:b1]
        if int(cb.sum()) == 0:
            continue
        first = int(coarse_start[b0])
        last = int(coarse_start[b1 - 1] + counts0[b1 - 1])
        max_n, max_l = int(cb.max()), int(lb.max())
        if len(cb) * max_n * max_l > SCORE_BUDGET or max_l > max_n:
            # buckets solved one by one (:138-160)
            cursor = first
            for j, (size, nleaf, offset) in enumerate(
                zip(cb.tolist(), lb.tolist(), leaf_start[b0:b1].tolist())
            ):
                if not size:
                    continue
                ids = order[cursor : cursor + size]
                cursor += size
                x = keys[ids]
                c = _solve_bucket_alone(
                    x, size, nleaf, local_iters, seed + 0x48494552 + b0 + j
                )
                cent[offset : offset + nleaf] = c
                rows = score_rows(nleaf)
                for start in range(0, size, rows):
                    labels[ids[start : start + rows]] = (
                        x[start : start + rows] @ c.t()
                    ).topk(spill, dim=1).indices + offset
                alone += 1
            continue

        # the batch padded into one slab (:161-173)
        ids = order[first:last]
        local_bucket = coarse[ids] - b0
        local_start = cb.cumsum(0) - cb
        rank = torch.arange(ids.numel(), device=dev) - torch.repeat_interleave(
            local_start, cb
        )
        rows_i = torch.arange(max_n, device=dev)
        cols_i = torch.arange(max_l, device=dev)
        row_ok = rows_i[None, :] < cb[:, None]
        col_ok = cols_i[None, :] < lb[:, None]

        xb = torch.zeros(b1 - b0, max_n, d, dtype=keys.dtype, device=dev)
        xb[local_bucket, rank] = keys[ids]
        # Seed leaves with random real keys (padding rows sort last); a
        # singleton bucket reuses its key for every extra leaf (:174-185).
        seed_rows = (
            torch.rand(b1 - b0, max_n, generator=gen)
            .to(dev)
            .masked_fill(~row_ok, torch.inf)
            .topk(max_l, dim=1, largest=False)
            .indices
        )
        seed_rows = torch.where(col_ok & (cols_i >= cb[:, None]), seed_rows[:, :1], seed_rows)
        cf = xb.gather(1, seed_rows[..., None].expand(-1, -1, d)).clone()

        for _ in range(local_iters):  # batched Lloyd steps (:187-199)
            score = torch.bmm(xb, cf.transpose(1, 2)).masked_fill(
                ~col_ok[:, None, :], -torch.inf
            )
            lab = score.argmax(2)
            if dev.type == "cpu":
                sums = torch.zeros_like(cf)
                sums.scatter_add_(1, lab[..., None].expand(-1, -1, d), xb * row_ok[..., None])
            else:
                sums = fixed_row_sums(max_l, lab, xb * row_ok[..., None], dim=1)
            cnt = torch.zeros(b1 - b0, max_l, dtype=keys.dtype, device=dev)
            cnt.scatter_add_(1, lab, row_ok.to(keys.dtype))
            cf = torch.where(cnt[..., None] > 0, sums / cnt[..., None].clamp_min(1), cf)
            cf = cf / cf.norm(dim=2, keepdim=True).clamp_min(EPS)

        # final labels against the updated codebook, leaves written back (:201-217)
        score = torch.bmm(xb, cf.transpose(1, 2)).masked_fill(
            ~col_ok[:, None, :], -torch.inf
        )
        top = score.topk(spill, dim=2).indices
        labels[ids] = top[local_bucket, rank] + leaf_start[coarse[ids], None]

        owner = torch.repeat_interleave(torch.arange(b1 - b0, device=dev), lb)
        owner_start = lb.cumsum(0) - lb
        local_leaf = torch.arange(int(lb.sum()), device=dev) - torch.repeat_interleave(
            owner_start, lb
        )
        cent[leaf_start[b0:b1][owner] + local_leaf] = cf[owner, local_leaf]

    # CSR posting lists and build statistics (:219-236)
    flat = labels.reshape(-1)
    key_of = torch.arange(n, device=dev).unsqueeze(1).expand_as(labels).reshape(-1)
    # a GPU sort is asked for stability outright (equal leaves keep key order)
    list_order = torch.argsort(flat) if dev.type == "cpu" else torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=n_leaves)
    offsets = torch.cat([torch.zeros(1, dtype=torch.long, device=dev), counts.cumsum(0)])
    stats = {
        "algorithm": "hierarchical",
        "coarse_clusters": k0,
        "coarse_score_pairs": n * k0 * coarse_iters,
        "local_score_pairs": int((counts0 * leaves).sum()) * (local_iters + 1),
        "legacy_score_pairs": n * n_leaves * max(1, local_iters + 1),
    }
    if alone:
        stats["chunked_buckets"] = alone
    return cent, key_of[list_order].int(), offsets, counts, labels, stats
