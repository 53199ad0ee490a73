"""Index codec, NPZ v4 archive and the query-independent key codec.

Host-side prefill code.  The formats must stay byte-compatible with the
reference so that an index dumped by either implementation loads in the other:

* ``pack2``/``unpack2`` — four 2-bit codes per byte, little-endian within the
  byte (reference ``_codecs/index.py:25-31``).
* ``encode_group_scale_cell`` — scale-sorted centroids, one scale per
  32-centroid group, 4-bit mid-rise codes split into an upper and a lower
  2-bit plane, CSR remapped with its centroids (reference
  ``_codecs/index.py:233-313``).
* NPZ version 4 — per-cell arrays ``"{i}_{name}"``, BF16 stored as int16 with a
  ``bf16_arrays`` manifest, JSON metadata (reference ``_codecs/index.py:130-230``).
* ``key_codec`` — per (KV head, coordinate) max-abs scale over every token and
  an 8-bit mid-rise code per coordinate (reference ``_codecs/keys.py:16-26``).
"""

from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path
from tempfile import NamedTemporaryFile

import numpy as np
import torch

LEGACY_VERSION = 3
INDEX_VERSION = 4
GROUP = 32
GROUP_CODEC = f"group-scale-{GROUP}-v1"
QUERY_FIELDS = frozenset({"q", "query_hash", "coarse_ids", "head_mask"})


def fingerprint(t: torch.Tensor) -> str:
    """SHA-256 of the tensor's raw bytes (reference ``_codecs/index.py:19-22``)."""
    raw = t.contiguous().view(torch.uint8).cpu().numpy()
    return hashlib.sha256(raw.tobytes()).hexdigest()


def pack2(codes: torch.Tensor) -> torch.Tensor:
    """[..., 4n] codes in 0..3 -> [..., n] bytes, code 4i+j in bits 2j..2j+1."""
    x = codes.to(torch.int64).reshape(*codes.shape[:-1], -1, 4)
    shifts = torch.tensor([0, 2, 4, 6], dtype=torch.int64)
    return (x << shifts).sum(-1).to(torch.uint8)


def unpack2(data: torch.Tensor) -> torch.Tensor:
    x = data.to(torch.int64).unsqueeze(-1) >> torch.tensor([0, 2, 4, 6])
    return (x & 3).flatten(-2)


def coarse_metadata(source: torch.Tensor, upper: torch.Tensor, scale: torch.Tensor):
    """Odd 2-bit coarse operands and the residual norm the coarse interval
    margin uses (reference ``_coarse_metadata`` ``_codecs/index.py:34-49``):
    the residual is measured against the *unrounded* 2-bit reconstruction
    ``scale * (2u - 3) / 4`` before FP16 storage."""
    odd = 2 * unpack2(upper).float() - 3
    full = scale.float().unsqueeze(-1) * odd / 4
    return dict(
        coarse2=full.half(),
        coarse_odd=odd.bfloat16(),
        coarse_residual_norm=(source.float() - full).norm(dim=-1).half(),
    )


def ensure_coarse_metadata(cell: dict) -> dict:
    """Derive missing coarse operands of a version-1 fixture in memory."""
    if all(k in cell for k in ("coarse2", "coarse_odd", "coarse_residual_norm")):
        return cell
    source = cell.get("coarse_centroids", cell["centroids"])
    if "scale" not in cell:
        cell = dict(
            cell, scale=(source.float().abs().amax(-1) * (16 / 15)).clamp_min(1e-9)
        )
    return dict(cell, **coarse_metadata(source, cell["upper"], cell["scale"]))


def require_group_scale_cell(cell: dict, group: int = GROUP) -> dict:
    """Check the persisted 32-centroid scale summary (reference ``:67-88``)."""
    if cell.get("summary_codec") != f"group-scale-{group}-v1" or (
        cell.get("group_scale_size") != group
    ):
        raise ValueError(
            "Stage-I index is not pre-grouped; regenerate it with "
            "SeoulKV4Index.build"
        )
    nc = len(cell["centroids"])
    if nc % group:
        raise ValueError("grouped Stage-I index has a partial centroid group")
    compact = cell.get("group_fine_scale")
    if not isinstance(compact, torch.Tensor) or compact.shape != (nc // group,):
        raise ValueError("grouped Stage-I index has an invalid compact scale table")
    full = cell.get("fine_scale")
    if not isinstance(full, torch.Tensor) or full.shape != (nc,):
        raise ValueError("grouped Stage-I index is missing its per-centroid scale view")
    if not torch.equal(full.reshape(-1, group), compact[:, None].expand(-1, group)):
        raise ValueError("grouped Stage-I index scale views disagree")
    return cell


def expand_lists(cell: dict, selected) -> torch.Tensor:
    """Sorted set of tokens posted under the selected clusters (``:91-94``)."""
    off, vals = cell["offsets"].long(), cell["values"].long()
    parts = [vals[off[int(c)] : off[int(c) + 1]] for c in selected]
    return torch.cat(parts).unique(sorted=True) if parts else vals[:0]


def validate_static_cell(c: dict) -> None:
    """Index invariants (reference ``validate_static_cell`` ``:97-116``): every
    retrieval token sits in exactly ``spill`` distinct lists, CSR is monotone,
    sink/local tokens are never posted.  Violations raise ``AssertionError``,
    the reference's error type for these checks."""
    nc, d = c["centroids"].shape
    if d != 256 or not 0 < int(c["p"]) <= min(nc, 1536):
        raise AssertionError("index cell has an invalid shape or probe budget")
    if not torch.isfinite(c["centroids"].float()).all():
        raise AssertionError("index centroids must be finite")
    if c["upper"].shape != (nc, 64) or c["lower"].shape != (nc, 64):
        raise AssertionError("index centroid planes must be [nc, 64] bytes")
    if c["coarse2"].shape != (nc, d) or c["coarse_odd"].shape != (nc, d):
        raise AssertionError("index coarse operands have the wrong shape")
    norm = c["coarse_residual_norm"]
    if norm.shape != (nc,) or not torch.isfinite(norm.float()).all():
        raise AssertionError("index coarse residual norms are invalid")
    off, vals = c["offsets"].long(), c["values"].long()
    if len(off) != nc + 1 or off[0] != 0 or off[-1] != len(vals):
        raise AssertionError("index CSR offsets do not cover the posting values")
    if (off[1:] < off[:-1]).any():
        raise AssertionError("index CSR offsets are not monotone")
    context, r0, r1 = int(c["context"]), int(c["r0"]), int(c["r1"])
    if ((vals < 0) | (vals >= context)).any():
        raise AssertionError("index posting token outside the context")
    counts = torch.bincount(vals, minlength=context)
    if not (counts[r0:r1] == int(c["spill"])).all():
        raise AssertionError("every retrieval token must sit in exactly spill lists")
    if counts[:r0].sum() or counts[r1:].sum():
        raise AssertionError("sink/local tokens must not be posted")
    rows = torch.repeat_interleave(torch.arange(nc), off.diff())
    entries = (rows * context + vals).sort().values
    if (entries[1:] == entries[:-1]).any():
        raise AssertionError("a token is posted twice in one cluster")


def validate_cell(c: dict) -> None:
    """Legacy fixture check, including its replay query (``:119-127``)."""
    c = ensure_coarse_metadata(c)
    validate_static_cell(c)
    nc, d = c["centroids"].shape
    if c["q"].shape != (4, d) or not torch.isfinite(c["q"].float()).all():
        raise AssertionError("legacy fixture query is invalid")
    ids, mask = c["coarse_ids"].long(), c["head_mask"].long()
    if not len(ids) or (ids < 0).any() or (ids >= nc).any():
        raise AssertionError("legacy fixture coarse IDs are invalid")
    if (ids[1:] <= ids[:-1]).any() or ((mask <= 0) | (mask >= 16)).any():
        raise AssertionError("legacy fixture coarse IDs/masks are invalid")
    if any(int(((mask >> h) & 1).sum()) < int(c["p"]) for h in range(4)):
        raise AssertionError("legacy fixture head masks admit fewer than P centroids")


def load_index(path) -> tuple[list[dict], dict]:
    """Read a v4 index or a legacy v1-v3 grouped fixture (``:130-177``)."""
    with np.load(path, allow_pickle=False) as z:
        meta = json.loads(str(z["metadata"]))
        version = meta.get("version")
        if version not in (1, 2, LEGACY_VERSION, INDEX_VERSION):
            raise ValueError("unsupported Stage-I index version")
        static = version == INDEX_VERSION
        bf16 = set(meta.get("bf16_arrays", ())) if static else set()
        if not bf16.issubset(z.files):
            raise ValueError("Stage-I index is missing a declared BF16 array")
        cells = []
        for i, info in enumerate(meta["cells"]):
            cell = dict(info)
            prefix = f"{i}_"
            for name in z.files:
                if not name.startswith(prefix):
                    continue
                tensor = torch.from_numpy(z[name])
                if name in bf16:
                    if tensor.dtype != torch.int16:
                        raise ValueError(f"invalid BF16 storage for {name}")
                    tensor = tensor.view(torch.bfloat16)
                cell[name[len(prefix) :]] = tensor
            if static:
                if QUERY_FIELDS.intersection(cell):
                    raise ValueError("static Stage-I index contains replay query fields")
                validate_static_cell(cell)
            else:
                cell["q"] = cell["q"].bfloat16()
                cell = ensure_coarse_metadata(cell)
                validate_cell(cell)
            if version >= LEGACY_VERSION:
                cell = require_group_scale_cell(cell)
            cells.append(cell)
    return cells, meta


def _archive(cells, meta) -> dict:
    data, rows, bf16 = {}, [], []
    for i, cell in enumerate(cells):
        scalars = {}
        for name, value in cell.items():
            if name in QUERY_FIELDS:
                continue
            if isinstance(value, torch.Tensor):
                key = f"{i}_{name}"
                if value.dtype == torch.bfloat16:
                    # NumPy has no BF16: keep the raw words and declare them.
                    value = value.view(torch.int16)
                    bf16.append(key)
                data[key] = value.contiguous().numpy()
            else:
                scalars[name] = value
        rows.append(scalars)
    metadata = dict(meta, version=INDEX_VERSION, cells=rows, bf16_arrays=bf16)
    data["metadata"] = np.array(json.dumps(metadata))
    return data


def dump_index(path, cells, meta) -> None:
    """Write a query-free NPZ at ``path``; replace the file only on success."""
    path = Path(path)
    data = _archive(cells, meta)
    path.parent.mkdir(parents=True, exist_ok=True)
    temp = NamedTemporaryFile(dir=path.parent, prefix=f".{path.name}.", delete=False)
    try:
        with temp:
            np.savez(temp, **data)
        os.replace(temp.name, path)
    finally:
        Path(temp.name).unlink(missing_ok=True)


def encode_group_scale_cell(cell: dict, group: int = GROUP):
    """Sort centroids by range, quantize to 4-bit odd levels with one scale per
    ``group`` centroids, and move each posting list with its centroid.

    Returns ``(encoded_cell, inverse)`` where ``inverse[old] = new`` physical
    centroid index.  The arithmetic order follows the reference exactly
    (``_codecs/index.py:233-313``) because the codes are part of the index
    format: code = clamp(floor((c + s) / (s / 8)), 0, 15) and the decoded
    centroid is fp16(s * (2 code - 15) / 16).
    """
    if group <= 0 or group % 8:
        raise ValueError("group scale size must be a positive multiple of 8")
    original = cell.get("coarse_centroids", cell["centroids"])
    cen = original.float()
    nc, d = cen.shape
    if d != 256 or nc % group:
        raise ValueError(
            f"group-scale cell requires [multiple of {group},256], got {tuple(cen.shape)}"
        )
    ranges = cell.get("scale")
    if ranges is None:
        ranges = (cen.abs().amax(-1) * (16 / 15)).clamp_min(1e-9)
    perm = torch.argsort(ranges.float(), stable=True)
    cen = cen[perm]
    group_scale = (cen.reshape(-1, group, d).abs().amax(dim=(1, 2)) * (16 / 15)).clamp_min(
        1e-9
    )
    scale = group_scale.repeat_interleave(group)
    s = scale[:, None]
    code = ((cen + s) / (s / 8)).floor().clamp(0, 15).byte()
    odd = (2 * code.float() - 15).bfloat16()
    decoded = (s * odd.float() / 16).half()
    levels = (
        (group_scale[:, None, None] * (2 * torch.arange(16).float()[None, None] - 15) / 16)
        .expand(-1, group, -1)
        .reshape(nc, 16)
        .half()
    )
    upper, lower = pack2(code >> 2), pack2(code & 3)

    offsets = cell["offsets"].long()
    lengths = offsets[1:] - offsets[:-1]
    owner = torch.repeat_interleave(torch.arange(nc), lengths)
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(nc)
    # Stable: token order inside each list is preserved.
    posting_order = torch.argsort(inverse[owner], stable=True)
    new_offsets = torch.cat((torch.zeros(1, dtype=torch.long), lengths[perm].cumsum(0)))
    group_fine_scale = (group_scale / 16).half()
    encoded = dict(
        cell,
        coarse_centroids=cen.to(original.dtype),
        centroids=decoded.bfloat16(),
        upper=upper,
        lower=lower,
        scale=scale,
        decoded=decoded.bfloat16(),
        fine_scale=group_fine_scale.repeat_interleave(group),
        group_fine_scale=group_fine_scale,
        levels=levels,
        centroid_codec="fp16-scale-odd-v1",
        offsets=new_offsets.to(cell["offsets"].dtype),
        values=cell["values"][posting_order],
        max_codec_error=float((cen - decoded.float()).abs().max()),
        group_scale_size=group,
        summary_codec=f"group-scale-{group}-v1",
        **coarse_metadata(cen, upper, scale),
    )
    return encoded, inverse


def key_codec(k: torch.Tensor) -> dict:
    """8-bit mid-rise key codes over all tokens of each KV head.

    ``scales[g, d] = max_t |K[g, t, d]|`` (clamped to 1e-9) and
    ``code8 = clamp(floor((K + s) / (2 s / 256)), 0, 255)`` in fp32
    (reference ``_stage15_key_codec`` ``_codecs/keys.py:16-26``).  The device
    key planes are the bit fields of ``code8``: bits 7..6 (Stage-1.5 prefix),
    bits 5..4 (Stage-1.6 residual) and bits 3..0 (Stage-II residual).
    """
    kf = k.float()
    scales = kf.abs().amax(dim=1).clamp_min(1e-9)
    step8 = 2 * scales[:, None, :] / 256
    code8 = torch.clamp(torch.floor((kf + scales[:, None, :]) / step8), 0, 255)
    return {"code8": code8.to(torch.uint8).contiguous(), "scales": scales.contiguous()}


def pack_lowbits(values: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack ``8 // bits`` codes per byte, little-endian (``_codecs/keys.py:6-13``)."""
    per = 8 // bits
    if values.shape[-1] % per:
        raise ValueError("head dimension is not packable")
    grouped = values.to(torch.int16).reshape(*values.shape[:-1], -1, per)
    shifts = torch.arange(per, dtype=torch.int16) * bits
    return (grouped << shifts).sum(dim=-1).to(torch.uint8).contiguous()


def encode_planes(code8: torch.Tensor) -> dict:
    """The reference's three key planes of ``code8`` [G, T, 256] (``:29-44``)."""
    return {
        "prefix2": pack_lowbits(code8 >> 6, 2),
        "residual2": pack_lowbits((code8 >> 4) & 3, 2),
        "residual4": pack_lowbits(code8 & 15, 4),
    }
