"""GPU tests of the operator boundary: cache outputs (omitted / bound onto the inputs / buffers of
their own), device-only metadata (no host copies: the query-length bound picks the kernels),
malformed device metadata (kernels clamp every index: the call ends normally with bounded
outputs), and the append's block-table last-writer scan over more than 256 sequences.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16
from pa_cases import make_case, run_gpu_op

pytestmark = pytest.mark.gpu


def _outputs_match(case, out, tol=2e-3):
    ref, ref_t, _, _ = orc.paged_attention_op(case)
    dt = case["dtype"]
    got = orc.decode(out, dt).astype(np.float64)
    err = orc.rel_l2(got, orc.decode(ref_t, dt))
    assert err <= tol, f"rel-L2 vs T-rounded oracle {err:.3e}"
    assert orc.rel_l2(got, ref) <= 2 * tol


# test_paged_attention.py:492-602: outputs 1/2 omitted, separate or aliased, with and without a
# slot_mapping remap, over the reference's two geometries and seeds (the single-sequence geometry
# keeps one token for seeds 87/89 and, for seed 89 with a remap, writes slot 0 of its first block)
@pytest.mark.parametrize("outputs", ["omitted", "separate", "aliased"])
@pytest.mark.parametrize("remap", [False, True])
@pytest.mark.parametrize("geometry", [(4, 2, 16, 16, 4, 2), (24, 4, 256, 5, 256, 1)],
                         ids=["small", "head256"])
def test_partial_cache_writeback(outputs, remap, geometry):
    H, KV, d, nb, block, batch = geometry
    for seed in (87, 88, 89):
        case = make_case(H, KV, d, nb, block, batch, dtype=F16, seed=seed)
        if batch == 1 and seed != 88:
            for name in ("query", "key", "value"):
                case[name] = case[name][:1]
            case["cum"] = np.array([0, 1], np.int32)
        if remap:
            nt = int(case["cum"][-1])
            slots = np.random.default_rng(seed).permutation(nb * block)[:nt].astype(np.int32)
            slots[0] = (int(case["block_table"][0, 0]) * block
                        if batch == 1 and seed == 89 else -1)
            case["slot_mapping"] = slots
        ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
        res = run_gpu_op(case, cache_outputs=outputs)
        out, kc, vc = res[:3]
        got = orc.decode(out, F16).astype(np.float64)
        assert orc.rel_l2(got, orc.decode(ref_t, F16)) <= 2e-3, seed
        # the output caches (or, when omitted / aliased, the inputs) hold the updated caches
        assert np.array_equal(kc, kc_ref) and np.array_equal(vc, vc_ref), seed
        if outputs == "separate":  # the inputs were updated in place as well
            assert np.array_equal(res[3], kc_ref) and np.array_equal(res[4], vc_ref), seed


def test_latent_rejects_value_cache_output():
    import torch
    from onnxruntime_ep_mlx_amd import PagedAttentionError
    from pa_cases import make_latent_case
    case = make_latent_case(4, 64, 32, 8, 16, 2, dtype=BF16, seed=5)
    with pytest.raises((PagedAttentionError, ValueError)):
        import onnxruntime_ep_mlx_amd as ep
        from pa_cases import to_torch
        kc = to_torch(case["key_cache"], BF16)
        I = lambda k: torch.from_numpy(case[k]).cuda()
        ep.paged_attention(to_torch(case["query"], BF16), to_torch(case["key"], BF16), None, kc,
                           None, I("cum"), I("past"), I("block_table"), num_heads=4,
                           kv_num_heads=1, v_head_size=32, kv_cache_layout="LATENT",
                           value_cache_out=torch.empty_like(kc))


# Device-only metadata (validate=False: no host copies).  A decode batch with max_query_len = 1
# takes the balanced decode; the same batch with no bound (read as num_tokens) takes the prefill
# kernel; a prefill batch with its bound; all against the oracle, caches bit-exact.
@pytest.mark.parametrize("mq", [1, 0], ids=["bound1", "unbounded"])
def test_device_only_metadata_decode(mq):
    rng = np.random.default_rng(303)
    B, bs = 16, 16
    ctx = rng.integers(512, 2049, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    case = make_case(32, 8, 128, B * mb, bs, B, dtype=BF16, seed=303, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=mb, do_rotary=1, theta=500000.0, std=1.0)
    _, _, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case, validate=False, max_query_len=mq)
    assert np.array_equal(kc, kc_ref) and np.array_equal(vc, vc_ref)
    _outputs_match(case, out)


def test_device_only_metadata_prefill():
    rng = np.random.default_rng(304)
    B, bs = 6, 16
    new = np.array([64, 1, 33, 64, 0, 17])
    past = rng.integers(0, 900, size=B)
    mb = int((past.max() + new.max() + bs - 1) // bs)
    case = make_case(28, 4, 128, B * mb, bs, B, dtype=BF16, seed=304, new_lens=new, past=past,
                     max_blocks=mb, std=1.0)
    _, _, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case, validate=False, max_query_len=64)
    assert np.array_equal(kc, kc_ref) and np.array_equal(vc, vc_ref)
    _outputs_match(case, out)


def test_max_query_len_checked_against_host_metadata():
    from onnxruntime_ep_mlx_amd import PagedAttentionError
    case = make_case(8, 2, 64, 16, 16, 2, dtype=F16, seed=9, new_lens=[3, 1], past=[4, 9],
                     max_blocks=8)
    with pytest.raises(PagedAttentionError, match="max_query_len"):
        run_gpu_op(case, validate=True, max_query_len=2)


# Malformed device metadata, not validated on the host: block ids outside the pool (negative and
# too large) and a past length beyond the block table's capacity.  Every kernel clamps its page
# ids and positions, so the call completes; the new rows of the malformed sequences have no valid
# slot and are not written, and the well-formed sequences are unaffected.  Outputs of malformed
# sequences are convex combinations of cache rows: finite and bounded by the largest value.
@pytest.mark.parametrize("mq,new", [(1, 1), (16, 16)], ids=["decode", "prefill"])
def test_malformed_device_metadata_is_contained(mq, new):
    B, bs, mb, nb = 4, 16, 8, 64
    case = make_case(8, 2, 128, nb, bs, B, dtype=BF16, seed=77 + new, new_lens=[new] * B,
                     past=[40, 70, 30, 50], max_blocks=mb, std=1.0)
    good = make_case(8, 2, 128, nb, bs, B, dtype=BF16, seed=77 + new, new_lens=[new] * B,
                     past=[40, 70, 30, 50], max_blocks=mb, std=1.0)
    bt = case["block_table"].copy()
    bt[2, :] = [-5, 1000, -1, nb, 7, nb + 3, -100, 2 ** 30]  # every id of sequence 2 invalid
    case["block_table"] = bt
    case["past"] = case["past"].copy()
    case["past"][3] = mb * bs + 500  # sequence 3 beyond its block table's capacity
    out, kc, vc = run_gpu_op(case, validate=False, max_query_len=mq)
    # the well-formed sequences 0 and 1 against the oracle run on them alone
    sub = dict(good)
    T01 = int(good["cum"][2])
    for name in ("query", "key", "value"):
        sub[name] = good[name][:T01]
    sub["cum"] = good["cum"][:3].copy()
    sub["past"] = good["past"][:2].copy()
    sub["block_table"] = good["block_table"][:2].copy()
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(sub)
    # sequences 2 and 3 wrote nothing: the pool equals the oracle's for sequences 0 and 1
    assert np.array_equal(kc, kc_ref) and np.array_equal(vc, vc_ref)
    got = orc.decode(out, BF16).astype(np.float64)
    assert orc.rel_l2(got[:T01], orc.decode(ref_t, BF16)) <= 2e-3
    bad = got[T01:]
    vmax = np.abs(orc.decode(case["value_cache"], BF16)).max()
    vmax = max(vmax, np.abs(orc.decode(case["value"], BF16)).max())
    assert np.all(np.isfinite(bad)) and np.abs(bad).max() <= vmax * 1.01


# The append's block-table last-writer scan over more than 256 sequences: sequence pairs whose
# new positions land on one slot, near each other and across the 256-sequence chunks of the scan.
def test_block_table_duplicates_beyond_256_sequences():
    B, bs, mb = 300, 16, 4
    rng = np.random.default_rng(300)
    past = rng.integers(0, mb * bs - 1, size=B)
    case = make_case(8, 2, 64, B * mb, bs, B, dtype=BF16, seed=300, new_lens=[1] * B, past=past,
                     max_blocks=mb, std=1.0)
    bt = case["block_table"].copy()
    for a, b in ((3, 280), (10, 11), (200, 299), (255, 256), (0, 150)):
        # b's new position lands on a's new slot: same block id and same offset in the block
        past[b] = past[a]
        bt[b, past[b] // bs] = bt[a, past[a] // bs]
    case["past"] = past.astype(np.int32)
    case["block_table"] = bt
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case)
    assert np.array_equal(kc, kc_ref) and np.array_equal(vc, vc_ref)
    got = orc.decode(out, BF16).astype(np.float64)
    assert orc.rel_l2(got, orc.decode(ref_t, BF16)) <= 2e-3
