"""Pins every stage of the oracle decode step (``oracle/decode.py``) on a
config-0 sized case, by means independent of the oracle's own formulas:

* score stages against float64 evaluations of the reference's *own* operand
  forms (its decoded index fields, its key planes, its two-term 8-bit form);
* selections against brute-force full sorts with the (score desc, lowest ID)
  rule and the reference's invariants;
* the pool against literal restatements of the reference's ``encounter_union``
  and ``local_encounter_union`` loops (``_kernels/common/seoulkv4_cluster_blocks.py``);
* attention against ``torch.nn.functional.scaled_dot_product_attention``.

CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits, case, oracle_inputs, oracle_step
from oracle import arith
from oracle import decode as od

PARAMS = dict(context=8192, components=256, nc=512, nprobe=64)


@pytest.fixture(scope="module")
def step():
    index, k, v, qs = case(**PARAMS)
    traces, out = oracle_step(PARAMS, qs[0])
    return index, k, v, qs[0], traces, out


def bf16_f64(b):
    return arith.bf16_to_f32(b).astype(np.float64)


def ulp_bf16(x):
    """Spacing of BF16 values at |x| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_bf16_near(got_bits, ref, slack=0.0):
    """BF16 result within one BF16 ulp of the exact value plus ``slack``
    (the FP32 intermediate roundings of the canonical arithmetic)."""
    got = bf16_f64(got_bits)
    err = np.abs(got - ref)
    tol = ulp_bf16(ref) + slack
    assert (err <= tol).all(), float((err - tol).max())
    # and the vast majority are the correctly rounded BF16 of the exact value
    exact = bf16_f64(arith.bf16_bits(ref.astype(np.float32)))
    assert np.mean(got == exact) > 0.97


# ----------------------------------------------------------------- key codec
def _torch_key_codec(k):
    # the reference's expression order, evaluated by torch (_codecs/keys.py:16-26)
    kf = k.float()
    scales = kf.abs().amax(dim=1).clamp_min(1e-9)
    step8 = 2 * scales[:, None, :] / 256
    code8 = torch.clamp(torch.floor((kf + scales[:, None, :]) / step8), 0, 255).to(torch.uint8)
    return code8.numpy(), scales.numpy()


def test_key_codec_matches_torch_closed_form(step):
    _, k, *_ = step
    code8, scales = od.key_codec(bits(k))
    want_code, want_scales = _torch_key_codec(k)
    assert np.array_equal(scales, want_scales)
    assert np.array_equal(code8, want_code)
    # bucket invariants: monotone in K per coordinate; the extreme key of each
    # coordinate lands in the top bucket (clamped 256 -> 255)
    kf = k.float().numpy()
    g, d = 1, 17
    order = np.argsort(kf[g, :, d], kind="stable")
    assert (np.diff(code8[g, order, d].astype(int)) >= 0).all()
    assert code8[g, np.argmax(np.abs(kf[g, :, d])), d] in (0, 255)


def test_product_host_codec_matches_oracle(step):
    from seoulkv_amd import _codecs

    _, k, *_ = step
    codec = _codecs.key_codec(k)
    code8, scales = od.key_codec(bits(k))
    assert np.array_equal(codec["code8"].numpy(), code8)
    assert np.array_equal(codec["scales"].numpy(), scales)


# ----------------------------------------------------------------- query prep
def test_query_prep(step):
    index, k, _, q, *_ = step
    _, code8, scales, *_ = oracle_inputs(**PARAMS)
    qg = q.reshape(4, 4, 256).bfloat16()
    for g in range(4):
        qp = od.prepare_query(bits(qg[g]), scales[g], index.cells[g]["lam"])
        s = torch.from_numpy(scales[g])
        q15 = (qg[g].float() * s[None] / 64).bfloat16()
        qsv = (qg[g].float() * s[None] / 256).bfloat16()
        assert np.array_equal(qp.q15_bits, bits(q15))
        assert np.array_equal(qp.qs_bits, bits(qsv))
        norm64 = np.linalg.norm(qg[g].double().numpy(), axis=-1) * index.cells[g]["lam"]
        assert np.allclose(qp.norm, norm64, rtol=2.0 ** -22, atol=0)


# ------------------------------------------------------------- coarse / fine
def test_coarse_intervals_against_decoded_index_fields(step):
    index, _, _, q, traces, _ = step
    qg = q.reshape(4, 4, 256).double().numpy()
    for g in range(4):
        c = index.cells[g]
        odd = c["coarse_odd"].double().numpy()                  # 2u - 3, from the index
        scale = c["scale"].double().numpy()
        resid = c["coarse_residual_norm"].bfloat16().double().numpy()
        norm = np.linalg.norm(qg[g], axis=-1) * c["lam"]
        value = (qg[g] @ odd.T) * scale[None] / 4
        margin = norm[:, None] * resid[None]
        slack = 2.0 ** -21 * (np.abs(value) + margin)
        assert_bf16_near(traces[g].lower, value - margin, slack)
        assert_bf16_near(traces[g].upper, value + margin, slack)


def test_fine_scores_against_decoded_centroids(step):
    index, _, _, q, traces, _ = step
    qg = q.reshape(4, 4, 256).double().numpy()
    for g in range(4):
        c = index.cells[g]
        ids = traces[g].survivors
        # decoded = fp16(s (2 code - 15) / 16) carries its own FP16 rounding:
        # bound it by |q| . |decoded| 2^-11
        dec = c["decoded"].double().numpy()[ids]
        gfs = c["group_fine_scale"].double().numpy()[ids // 32]
        gs = c["scale"].double().numpy()[ids]
        ref = (qg[g] @ dec.T) * (gfs * 16 / gs)[None]
        slack = (np.abs(qg[g]) @ np.abs(dec).T) * 2.0 ** -10 + 2.0 ** -20 * np.abs(ref)
        got = bf16_f64(traces[g].fine)
        assert (np.abs(got - ref) <= ulp_bf16(ref) + slack).all()


# ----------------------------------------------------------------- selections
def test_thresholds_and_survivors_brute_force(step):
    index, *_, traces, _ = step
    for g in range(4):
        tr, p = traces[g], index.cells[g]["p"]
        lower, upper = bf16_f64(tr.lower), bf16_f64(tr.upper)
        assert not np.any(tr.upper == 0x8000) and not np.any(tr.lower == 0x8000)
        for h in range(4):
            thr = sorted(lower[h], reverse=True)[p - 1]
            assert float(bf16_f64(np.array([_unorder(tr.thr[h])]))[0]) == thr
            surv = {c for c in range(len(upper[h])) if upper[h][c] >= thr}
            got = {int(c) for c in np.flatnonzero((tr.masks >> h) & 1)}
            assert got == surv
            assert len(surv) >= p  # every head keeps at least P survivors
        assert np.array_equal(tr.survivors, np.flatnonzero(tr.masks))


def _unorder(o):
    o = int(o)
    return o ^ 0x8000 if o & 0x8000 else (~o) & 0xFFFF


def test_fine_select_brute_force(step):
    index, *_, traces, _ = step
    for g in range(4):
        tr, p = traces[g], index.cells[g]["p"]
        fine = bf16_f64(tr.fine)
        want = set()
        for h in range(4):
            elig = [i for i in range(len(tr.survivors)) if (tr.masks[tr.survivors[i]] >> h) & 1]
            best = sorted(elig, key=lambda i: (-fine[h][i], tr.survivors[i]))[:p]
            want |= {int(tr.survivors[i]) for i in best}
        assert tr.selected.tolist() == sorted(want)
        assert set(tr.selected.tolist()) <= set(tr.survivors.tolist())


# ----------------------------------------------------------------------- pool
def _mates(cell):
    off, vals = cell["offsets"].long().tolist(), cell["values"].long().tolist()
    where = {}
    for c in range(len(off) - 1):
        for j in range(off[c], off[c + 1]):
            where.setdefault(vals[j], []).append(c)
    mate = []
    for c in range(len(off) - 1):
        for j in range(off[c], off[c + 1]):
            other = [x for x in where[vals[j]] if x != c]
            assert len(where[vals[j]]) <= 2 and len(other) == len(where[vals[j]]) - 1
            mate.append(other[0] if other else None)
    return mate


def _encounter_union(cell, selected):
    """Literal restatement of the reference's first-occurrence loop."""
    off, vals = cell["offsets"].tolist(), cell["values"].tolist()
    seen, out = set(), []
    for cid in selected:
        for t in vals[off[cid] : off[cid + 1]]:
            if t not in seen:
                seen.add(t)
                out.append(t)
    return out


def _owner_union(cell, selected, mates, workers):
    """Mate-ownership form, split over ``workers`` contiguous ranges."""
    off, vals = cell["offsets"].tolist(), cell["values"].tolist()
    rank = {}
    for i, c in enumerate(selected):
        rank.setdefault(c, i)
    out = []
    for w in range(workers):
        for i in range(len(selected) * w // workers, len(selected) * (w + 1) // workers):
            c = selected[i]
            out.extend(vals[j] for j in range(off[c], off[c + 1])
                       if rank.get(mates[j], len(selected)) > i)
    return out


def test_pool_matches_encounter_union_and_ownership(step):
    index, *_, traces, _ = step
    rng = np.random.default_rng(5)
    for g in range(2):
        cell = index.cells[g]
        gc = od.GroupCell.from_cell(cell)
        mates = _mates(cell)
        nc = len(cell["offsets"]) - 1
        sets = [traces[g].selected.tolist(), [], list(range(nc)),
                sorted(rng.choice(nc, 37, replace=False).tolist())]
        for sel in sets:
            want = _encounter_union(cell, sel)
            assert od.pool(gc, np.array(sel, dtype=np.int64)).tolist() == want
            assert _owner_union(cell, sel, mates, 24) == want
            assert _owner_union(cell, sel, mates, 1) == want
        assert len(traces[g].pool) == len(set(traces[g].pool.tolist()))


# --------------------------------------------------------- stage 1.5/1.6/II
def _planes(code8g, tokens):
    c = code8g[tokens].astype(np.int64)
    return c >> 6, (c >> 4) & 3, c & 15   # prefix2, residual2, residual4


def test_refinement_scores_against_reference_operand_forms(step):
    index, _, _, q, traces, _ = step
    _, code8, scales, *_ = oracle_inputs(**PARAMS)
    qg = q.reshape(4, 4, 256).bfloat16()
    for g in range(4):
        tr = traces[g]
        s = torch.from_numpy(scales[g])
        q15 = (qg[g].float() * s[None] / 64).bfloat16()
        qsv = (qg[g].float() * s[None] / 256).bfloat16()
        q15x16 = (16 * q15.float()).bfloat16().double().numpy()
        qsx16 = (16 * qsv.float()).bfloat16().double().numpy()
        qs1 = qsv.double().numpy()
        p2, r2, r4 = _planes(code8[g], tr.pool)
        assert_bf16_near(tr.s2, q15x16 @ (2 * p2 - 3).T.astype(np.float64))
        p2, r2, r4 = _planes(code8[g], tr.u1)
        code4 = (p2 << 2) | r2
        assert_bf16_near(tr.s4, qsx16 @ (2 * code4 - 15).T.astype(np.float64))
        p2, r2, r4 = _planes(code8[g], tr.u2)
        code4 = (p2 << 2) | r2
        two_term = qsx16 @ (2 * code4 - 15).T.astype(np.float64) + qs1 @ (2 * r4 - 15).T
        assert_bf16_near(tr.s8, two_term)


def _brute_top(scores_bits, tokens, k):
    f = bf16_f64(scores_bits)
    return [sorted(range(len(tokens)), key=lambda i: (-f[h][i], tokens[i]))[:k]
            for h in range(f.shape[0])]


def test_funnel_unions_and_topk_brute_force(step):
    *_, traces, _ = step
    for g in range(4):
        tr = traces[g]
        assert not any(np.any(s == 0x8000) for s in (tr.s2, tr.s4, tr.s8))
        top = _brute_top(tr.s2, tr.pool.tolist(), od.M15_UNION)
        members = sorted({i for h in top for i in h})
        assert tr.u1.tolist() == [int(tr.pool[i]) for i in members]  # pool order
        assert len(tr.u1) <= 4 * od.M15_UNION
        top = _brute_top(tr.s4, tr.u1.tolist(), od.M16)
        members = sorted({i for h in top for i in h})
        assert tr.u2.tolist() == [int(tr.u1[i]) for i in members]  # U1 order
        top = _brute_top(tr.s8, tr.u2.tolist(), od.TOPK)
        assert tr.top100.tolist() == [[int(tr.u2[i]) for i in h] for h in top]


# ------------------------------------------------------------------ attention
def test_sdpa_matches_torch(step):
    *_, traces, out = step
    index, k, v, q, *_ = step
    _, _, _, k8, v8 = oracle_inputs(**PARAMS)
    qf = q.reshape(16, 256).float()
    for j in (0, 5, 10, 15):
        g, h = divmod(j, 4)
        ids = od.attention_ids(8192, 128, 256, traces[g].top100[h])
        assert len(ids) == 128 + 256 + 100 and len(set(ids.tolist())) == len(ids)
        kk = torch.from_numpy(k8[g][ids]).double()[None, None]
        vv = torch.from_numpy(v8[g][ids]).double()[None, None]
        want = torch.nn.functional.scaled_dot_product_attention(
            qf[j].double()[None, None, None], kk, vv
        )[0, 0, 0].numpy()
        assert np.allclose(out[j], want, rtol=1e-12, atol=1e-12)


def test_sparse_output_tracks_dense_decode(step):
    _, k, v, q, _, out = step
    dense = od.dense_decode(k.float().numpy(), v.float().numpy(), q.reshape(16, 256).float().numpy())
    cos = [float(out[j] @ dense[j] / np.linalg.norm(out[j]) / np.linalg.norm(dense[j]))
           for j in range(16)]
    assert min(cos) > 0.99


def test_grown_cache_attends_appended_tokens(step):
    """A cache grown by n appended tokens (context T0 + n, local L + n, the
    prefill's codes and cells): the same top-100 as the prefill step, and
    torch's SDPA over sink + [T0 - L, T0 + n) + top-100 -- every appended
    token once, no retrieval token twice."""
    _, _, _, q, traces, _ = step
    cells, code8, scales, k8, v8 = oracle_inputs(**PARAMS)
    n = 40
    gen = torch.Generator().manual_seed(5)
    kn = (torch.randn(4, n, 256, generator=gen) * 3).bfloat16()
    vn = torch.randn(4, n, 256, generator=gen).bfloat16()
    k8n, v8n = od.fp8_records(bits(kn), bits(vn))
    k8g, v8g = np.concatenate([k8, k8n], 1), np.concatenate([v8, v8n], 1)
    grown, out = od.decode_step(cells, code8, scales, k8g, v8g, bits(q).reshape(16, 256),
                                sink=128, local=256 + n, context=8192 + n)
    qf = q.reshape(16, 256).float()
    for g in range(4):
        np.testing.assert_array_equal(grown[g].top100, traces[g].top100)
    for j in (0, 7, 13):
        g, h = divmod(j, 4)
        ids = od.attention_ids(8192 + n, 128, 256 + n, grown[g].top100[h])
        assert set(range(8192, 8192 + n)) <= set(ids.tolist())
        assert len(set(ids.tolist())) == len(ids) == 128 + 256 + n + 100
        kk = torch.from_numpy(k8g[g][ids]).double()[None, None]
        vv = torch.from_numpy(v8g[g][ids]).double()[None, None]
        want = torch.nn.functional.scaled_dot_product_attention(
            qf[j].double()[None, None, None], kk, vv
        )[0, 0, 0].numpy()
        assert np.allclose(out[j], want, rtol=1e-12, atol=1e-12)


def test_dense_decode_matches_torch_sdpa():
    """``dense_decode`` (the CPU dense baseline and the dense FP8 path's
    reference) against torch's scaled_dot_product_attention in float64, GQA
    4:1 (query head j reads KV head j // 4), scale 1/sqrt(256)."""
    import torch

    g = torch.Generator().manual_seed(11)
    T = 3000
    k = torch.randn(4, T, 256, generator=g, dtype=torch.float32)
    v = torch.randn(4, T, 256, generator=g, dtype=torch.float32)
    q = torch.randn(16, 256, generator=g, dtype=torch.float32) * 0.5
    got = od.dense_decode(k.numpy(), v.numpy(), q.numpy())
    kk = k.double().repeat_interleave(4, dim=0)  # [16, T, 256]
    vv = v.double().repeat_interleave(4, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.double()[:, None, :], kk, vv, scale=1.0 / 16.0)[:, 0, :].numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-6)
    # a planted mistake (the GQA map j % 4) is caught
    bad = np.stack([
        (lambda lg: (np.exp(lg - lg.max()) / np.exp(lg - lg.max()).sum()) @ v.numpy()[j % 4])(
            k.numpy()[j % 4] @ q.numpy()[j] / 16.0) for j in range(16)])
    assert np.abs(bad - ref).max() > 1e-2
