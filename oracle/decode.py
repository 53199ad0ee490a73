"""CPU restatement of one SeoulKV4 sparse decode step (test infrastructure).

ORACLE — only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` may import this package, and only as the checker.

Every stage follows the reference algorithm; the score arithmetic is the
canonical one of ``oracle/arith.py``.  Stage map (reference file:line, paths
relative to ``src/seoulkv4/``):

=============  =============================================================
key_codec      ``_codecs/keys.py:16-26`` (code8, per-coordinate scales)
prepare_query  ``_kernels/query_prepare/host.py:26-51``
coarse         ``codegen/coarse_compute.py:61-119``,
               ``_kernels/stage1_coarse/seoulkv4_coarse_score.py:193-235``
threshold/     ``_kernels/stage1_coarse/seoulkv4_coarse_select.py:297-379``
survivors
fine           ``codegen/fine_postscale_codegen.py:6-71``, ``codegen/fine.py:1848-1861``
fine_select    ``_kernels/stage1_fine/seoulkv4_fine_native_select.py:35-73``
pool           ``codegen/stage15.py:275-345``, ``_kernels/common/seoulkv4_cluster_blocks.py:107-115``
score2/top     ``codegen/stage15.py:886-995,1027-1180``, ``_kernels/stage15/seoulkv4_stage15_matrix.py:10-19``
union U1       ``codegen/stage15.py:1519-1597``, ``_kernels/stage15/seoulkv4_stage15_union.py:4-25``
score4/top256  ``_kernels/stage16/seoulkv4_stage16_matrix.py:21-60``, ``codegen/refinement_fusion.py:232-266,402-455``
union U2       ``codegen/refinement_fusion.py:142-186``
score8/top100  ``_kernels/stage16/seoulkv4_union_matrix.py:49-139``, ``codegen/refinement_fusion.py:270-300,495-531``
sdpa           ``codegen/attention.py:35-201``, ``_runtime.py:76-95``,
               ``_kernels/stage16/seoulkv4_stage16_fused.py:1607`` (scale 1/16)
=============  =============================================================

Sizes follow the reference's fixed profile: 4 KV groups x 4 query heads,
d = 256, top-1600 of the Stage-1.5 frontier per head, top-256 in Stage 1.6,
top-100 in Stage II.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import arith

G = 4
H = 4
D = 256
M15_UNION = 1600
M15 = 2048
M16 = 256
TOPK = 100
ID_BITS_TOKEN = 20
ID_BITS_CENTROID = 16


def unpack2(packed: np.ndarray) -> np.ndarray:
    """[..., n] bytes -> [..., 4n] 2-bit codes, little-endian in each byte."""
    p = np.asarray(packed, dtype=np.uint8)[..., None]
    return ((p >> np.array([0, 2, 4, 6], dtype=np.uint8)) & 3).reshape(
        *p.shape[:-2], -1
    )


def key_codec(k_bits: np.ndarray):
    """``code8`` [G, T, 256] uint8 and ``scales`` [G, 256] fp32 of BF16 keys."""
    kf = arith.bf16_to_f32(k_bits)
    scales = np.maximum(np.abs(kf).max(axis=1), np.float32(1e-9)).astype(np.float32)
    step8 = ((np.float32(2) * scales) / np.float32(256)).astype(np.float32)
    code = np.floor(
        ((kf + scales[:, None, :]).astype(np.float32) / step8[:, None, :]).astype(np.float32)
    )
    return np.clip(code, 0, 255).astype(np.uint8), scales


@dataclass
class QueryPrep:
    X0: np.ndarray  # [H, D] fixed point of q (coarse / fine)
    fx0: np.ndarray  # [H]
    X15: np.ndarray  # of bf16(q s / 64)
    fx15: np.ndarray
    Xs: np.ndarray  # of bf16(q s / 256)
    fxs: np.ndarray
    norm: np.ndarray  # [H] fp32: ||q|| * lambda
    q15_bits: np.ndarray
    qs_bits: np.ndarray


def prepare_query(q_bits: np.ndarray, scales: np.ndarray, lam: float) -> QueryPrep:
    """Per-group query operands (``q_bits`` [4, 256] BF16 of one KV group)."""
    qb = np.asarray(q_bits, dtype=np.uint16)
    X0, fx0 = arith.fixed_point(qb)
    norm = np.array(
        [
            arith.f32_mul(
                arith.sqrt_rne_f32(int((X0[h] * X0[h]).sum()), int(fx0[h])),
                np.float32(lam),
            )
            for h in range(qb.shape[0])
        ],
        dtype=np.float32,
    )
    qf = arith.bf16_to_f32(qb)
    prod = arith.f32_mul(qf, scales[None, :])
    q15 = arith.bf16_bits((prod / np.float32(64)).astype(np.float32))
    qs = arith.bf16_bits((prod / np.float32(256)).astype(np.float32))
    X15, fx15 = arith.fixed_point(q15)
    Xs, fxs = arith.fixed_point(qs)
    return QueryPrep(X0, fx0, X15, fx15, Xs, fxs, norm, q15, qs)


def _centered_dot(X, codes, center):
    """exact sum_d X[h, d] * (2 codes[n, d] - center) -> [H, n] int64."""
    return 2 * arith.exact_dot(X, codes) - center * X.sum(axis=-1)[:, None]


@dataclass
class GroupCell:
    """Device-relevant view of one index cell."""

    upper: np.ndarray  # [nc, 256] codes 0..3 (bits 3..2 of the 4-bit code)
    lower: np.ndarray  # [nc, 256] codes 0..3
    scale4: np.ndarray  # [nc] fp32 = scale / 4
    resid: np.ndarray  # [nc] fp32 value of bf16(residual norm)
    gfs: np.ndarray  # [nc // 32] fp32 of the fp16 group fine scale
    offsets: np.ndarray  # [nc + 1] int64
    values: np.ndarray  # [postings] int64 token IDs
    p: int
    lam: float

    @classmethod
    def from_cell(cls, cell) -> "GroupCell":
        def np_(t):
            return t.contiguous().cpu().numpy()

        resid16 = np_(cell["coarse_residual_norm"]).view(np.uint16)
        return cls(
            upper=unpack2(np_(cell["upper"])),
            lower=unpack2(np_(cell["lower"])),
            scale4=(np_(cell["scale"]).astype(np.float32) / np.float32(4)).astype(np.float32),
            resid=arith.bf16_to_f32(arith.f16_bits_to_bf16_bits(resid16)),
            gfs=arith.f16_to_f32(np_(cell["group_fine_scale"]).view(np.uint16)),
            offsets=np_(cell["offsets"]).astype(np.int64),
            values=np_(cell["values"]).astype(np.int64),
            p=int(cell["p"]),
            lam=float(cell["lam"]),
        )


def coarse(cell: GroupCell, qp: QueryPrep):
    """Lower/upper BF16 interval bits [H, nc] of every centroid."""
    Dv = _centered_dot(qp.X0, cell.upper, 3)
    val = arith.to_f32(Dv, qp.fx0[:, None])
    value = arith.f32_mul(val, cell.scale4[None, :])
    margin = arith.f32_mul(qp.norm[:, None], cell.resid[None, :])
    lower = arith.bf16_bits(arith.f32_sub(value, margin))
    upper = arith.bf16_bits(arith.f32_add(value, margin))
    return lower, upper


def thresholds(lower: np.ndarray, p: int) -> np.ndarray:
    """P-th largest lower bound per head, as an ordered16 value."""
    o = np.sort(arith.ordered16(lower), axis=-1)[:, ::-1]
    return o[:, p - 1]


def survivor_masks(upper: np.ndarray, thr: np.ndarray) -> np.ndarray:
    """4-bit head mask per centroid: bit h iff upper_h >= threshold_h."""
    ok = arith.ordered16(upper) >= thr[:, None]
    return (ok.astype(np.int64) << np.arange(ok.shape[0])[:, None]).sum(axis=0)


def fine_scores(cell: GroupCell, qp: QueryPrep, ids: np.ndarray) -> np.ndarray:
    """BF16 bits [H, len(ids)] of the 4-bit rescoring of centroids ``ids``."""
    code4 = (cell.upper[ids].astype(np.int64) << 2) | cell.lower[ids]
    Dv = _centered_dot(qp.X0, code4, 15)
    val = arith.to_f32(Dv, qp.fx0[:, None])
    return arith.bf16_bits(arith.f32_mul(val, cell.gfs[ids // 32][None, :]))


def fine_select(scores, masks, ids, p) -> tuple[np.ndarray, list]:
    """Union over heads of each head's top-P eligible centroids, ascending."""
    per_head = []
    for h in range(scores.shape[0]):
        ok = ((masks >> h) & 1).astype(bool)
        keys = arith.topk_keys(arith.ordered16(scores[h][ok]), ids[ok], ID_BITS_CENTROID)
        per_head.append(np.sort(ids[ok][arith.top_k_by_key(keys, p)]))
    return np.unique(np.concatenate(per_head)), per_head


def pool(cell: GroupCell, selected: np.ndarray) -> np.ndarray:
    """Deduplicated candidate tokens in encounter order: selected clusters
    ascending, CSR order within a cluster, first occurrence kept."""
    if len(selected) == 0:
        return np.zeros(0, dtype=np.int64)
    parts = [cell.values[cell.offsets[c] : cell.offsets[c + 1]] for c in selected]
    tokens = np.concatenate(parts)
    _, first = np.unique(tokens, return_index=True)
    return tokens[np.sort(first)]


def scores_2bit(code8g, tokens, qp: QueryPrep):
    p2 = (code8g[tokens] >> 6).astype(np.int64)
    return arith.bf16_bits(arith.to_f32(_centered_dot(qp.X15, p2, 3), qp.fx15[:, None] + 4))


def scores_4bit(code8g, tokens, qp: QueryPrep):
    c4 = (code8g[tokens] >> 4).astype(np.int64)
    return arith.bf16_bits(arith.to_f32(_centered_dot(qp.Xs, c4, 15), qp.fxs[:, None] + 4))


def scores_8bit(code8g, tokens, qp: QueryPrep):
    c8 = code8g[tokens].astype(np.int64)
    return arith.bf16_bits(arith.to_f32(_centered_dot(qp.Xs, c8, 255), qp.fxs[:, None]))


def top_tokens(scores: np.ndarray, tokens: np.ndarray, k: int) -> list:
    """Per head: positions (into ``tokens``) of the top-k, best first."""
    out = []
    for h in range(scores.shape[0]):
        keys = arith.topk_keys(arith.ordered16(scores[h]), tokens, ID_BITS_TOKEN)
        out.append(arith.top_k_by_key(keys, k))
    return out


@dataclass
class GroupTrace:
    lower: np.ndarray
    upper: np.ndarray
    thr: np.ndarray
    masks: np.ndarray
    survivors: np.ndarray
    fine: np.ndarray
    selected: np.ndarray
    pool: np.ndarray
    s2: np.ndarray
    u1: np.ndarray
    s4: np.ndarray
    u2: np.ndarray
    s8: np.ndarray
    top100: np.ndarray  # [H, 100] token IDs, best first
    extra: dict = field(default_factory=dict)


def decode_group(cell: GroupCell, code8g: np.ndarray, qp: QueryPrep) -> GroupTrace:
    lower, upper = coarse(cell, qp)
    thr = thresholds(lower, cell.p)
    masks = survivor_masks(upper, thr)
    surv = np.flatnonzero(masks)
    fine = fine_scores(cell, qp, surv)
    selected, _ = fine_select(fine, masks[surv], surv, cell.p)
    pl = pool(cell, selected)
    s2 = scores_2bit(code8g, pl, qp)
    heads = top_tokens(s2, pl, M15_UNION)
    member = np.zeros(len(pl), dtype=bool)
    for pos in heads:
        member[pos] = True
    u1 = pl[member]  # pool order
    s4 = scores_4bit(code8g, u1, qp)
    heads = top_tokens(s4, u1, M16)
    member = np.zeros(len(u1), dtype=bool)
    for pos in heads:
        member[pos] = True
    u2 = u1[member]  # U1 order
    s8 = scores_8bit(code8g, u2, qp)
    heads = top_tokens(s8, u2, TOPK)
    top = np.stack([u2[pos] for pos in heads])
    return GroupTrace(lower, upper, thr, masks, surv, fine, selected, pl, s2, u1, s4, u2, s8, top)


def fp8_records(k_bits: np.ndarray, v_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """FP8 e4m3fn K and V as FP32 values (RNE cast from the BF16 values,
    overflow -> NaN), the build's stand-in for the reference's TT fp8_e4m3
    records (``_runtime.py:76-92``)."""
    import torch

    def cast(bits):
        t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
        return t.float().to(torch.float8_e4m3fn).float().numpy()

    return cast(k_bits), cast(v_bits)


def sdpa(q_f32: np.ndarray, k8: np.ndarray, v8: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """Softmax attention of one query row over the gathered FP8 rows, float64,
    scale 1/sqrt(256)."""
    kk = k8[ids].astype(np.float64)
    vv = v8[ids].astype(np.float64)
    logits = kk @ q_f32.astype(np.float64) / 16.0
    w = np.exp(logits - logits.max())
    return (w / w.sum()) @ vv


def attention_ids(context: int, sink: int, local: int, top: np.ndarray) -> np.ndarray:
    return np.concatenate(
        [np.arange(sink), np.arange(context - local, context), np.asarray(top, dtype=np.int64)]
    )


def decode_step(cells, code8, scales, k8, v8, q_bits, *, sink, local, context=None):
    """Full step.  ``cells``: 4 GroupCell; ``code8`` [4, T, 256]; ``scales``
    [4, 256]; ``k8``/``v8`` FP32 values of the FP8 records [4, T, 256];
    ``q_bits`` [16, 256] BF16 bits.  Returns (traces, out [16, 256] f64).
    ``context`` (default T): a cache grown by appended tokens after the
    prefill of T keys: ``k8``/``v8`` hold ``context`` rows, ``local`` is the
    grown window, while the codes, scales and cells stay the prefill's."""
    context = code8.shape[1] if context is None else context
    q_bits = np.asarray(q_bits, dtype=np.uint16).reshape(16, 256)
    traces, out = [], np.zeros((16, 256))
    for g in range(4):
        qp = prepare_query(q_bits[4 * g : 4 * g + 4], scales[g], cells[g].lam)
        tr = decode_group(cells[g], code8[g], qp)
        tr.extra["qprep"] = qp
        traces.append(tr)
        qf = arith.bf16_to_f32(q_bits[4 * g : 4 * g + 4])
        for h in range(4):
            ids = attention_ids(context, sink, local, tr.top100[h])
            out[4 * g + h] = sdpa(qf[h], k8[g], v8[g], ids)
    return traces, out


def dense_decode(k_f32: np.ndarray, v_f32: np.ndarray, q_f32: np.ndarray) -> np.ndarray:
    """Dense GQA decode over all T tokens (CPU baseline), fp32."""
    out = np.zeros((16, 256), dtype=np.float32)
    for j in range(16):
        g = j // 4
        logits = k_f32[g] @ q_f32[j] / np.float32(16)
        w = np.exp(logits - logits.max())
        out[j] = (w / w.sum()) @ v_f32[g]
    return out
