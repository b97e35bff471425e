"""The LATENT cache layout (kv_cache_layout = "LATENT", attention.rs:4058-4062, :4210-4213) on
the GPU through the C ABI, against the oracle: one kv head, no value input or value cache,
values = the first v_head_size dims of the rotated key rows, output [T, H * v_head_size].

Bars: key cache bytes bit-exact; outputs rel-L2 <= 2e-3 against the oracle rounded to T.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16
from pa_cases import make_latent_case, run_gpu_op

pytestmark = pytest.mark.gpu


def check_latent(case, tol=2e-3):
    print(f"latent case H={case['num_heads']} d={case['head_dim']} vd={case['v_head_size']}",
          flush=True)
    ref, _, kc_ref, _ = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case)
    assert vc is None
    np.testing.assert_array_equal(kc, kc_ref)
    got = orc.decode(out, case["dtype"]).astype(np.float64)
    want = orc.decode(orc.encode(ref.astype(np.float32), case["dtype"]),
                      case["dtype"]).astype(np.float64)
    err = orc.rel_l2(got, want)
    assert err <= tol, err


# test_paged_attention_latent_layout_and_rotary_offset (test_paged_attention.py:669-759)
def test_latent_reference_geometry():
    rng = np.random.default_rng(291)
    h, d, vd, nb, blk, nt, past_len = 2, 16, 8, 3, 4, 2, 3
    q = orc.encode(rng.standard_normal((nt, h * d)) * 0.2, F16)
    k = orc.encode(rng.standard_normal((nt, d)) * 0.2, F16)
    kc = orc.encode(rng.standard_normal((nb, blk, 1, d)) * 0.2, F16)
    half = 4
    inv = 1.0 / (10000.0 ** (np.arange(half) / half))
    ang = np.arange(nb * blk)[:, None] * inv[None, :]
    case = dict(num_heads=h, kv_num_heads=1, head_dim=d, dtype=F16, cache_dtype=F16,
                cum=np.array([0, nt], np.int32), past=np.array([past_len], np.int32),
                block_table=np.array([[1, 0, 2]], np.int32), query=q, key=k, key_cache=kc,
                cos_cache=orc.encode(np.cos(ang), F16), sin_cache=orc.encode(np.sin(ang), F16),
                rotary_offset=8, scale=0.2, latent=True, v_head_size=vd)
    check_latent(case)


@pytest.mark.parametrize("window,softcap,sink", [(-1, 0.0, False), (5, 0.0, False),
                                                 (-1, 0.8, True)])
def test_latent_masks_softcap_sink(window, softcap, sink):
    c = make_latent_case(4, 64, 48, 24, 4, 3, dtype=F16, seed=7, new_lens=[2, 1, 3],
                         past=[5, 0, 9], max_blocks=8, do_rotary=1, rot_dim=16,
                         rotary_offset=48, scale=0.125, window=window, softcap=softcap,
                         head_sink=np.linspace(-1, 1, 4) if sink else None)
    check_latent(c)


# MLA-sized latent heads: 576 = 512 latent + 64 rotary dims, values = the 512 latent dims
@pytest.mark.parametrize("new_lens", [[1, 1, 1], [5, 1, 9]], ids=["decode", "prefill"])
def test_latent_mla_sized_heads(new_lens):
    rng = np.random.default_rng(len(new_lens) + sum(new_lens))
    past = rng.integers(100, 700, 3)
    c = make_latent_case(16, 576, 512, 3 * 48, 16, 3, dtype=BF16, seed=int(past.sum()),
                         new_lens=new_lens, past=past, max_blocks=48, do_rotary=1, rot_dim=64,
                         rotary_offset=512, theta=10000.0, scale=float(1 / np.sqrt(192)),
                         std=1.0)
    check_latent(c)


# The LATENT matrix-core kernel (pa_latent.hip: four wavefronts split the score k-steps and the
# value dims of a 16-row block): MLA heads in both dtypes, 16 and 128 query heads, decode and
# ragged prefill batches, pages of 8 / 16 / 32 / 64 rows (8: rows addressed one by one), split
# contexts, softcap / window / sink, a negative scale, and values of 128 / 256 dims.
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("H", [16, 128])
@pytest.mark.parametrize("new_lens", [[1, 1, 1, 1], [7, 1, 33, 2]], ids=["decode", "prefill"])
def test_latent_mfma_mla(dtype, H, new_lens):
    rng = np.random.default_rng(H + len(new_lens) + sum(new_lens) + dtype)
    past = rng.integers(0, 700, 4)
    c = make_latent_case(H, 576, 512, 4 * 48, 16, 4, dtype=dtype, seed=int(past.sum()) + H,
                         new_lens=new_lens, past=past, max_blocks=48, do_rotary=1, rot_dim=64,
                         rotary_offset=512, theta=10000.0, scale=float(1 / np.sqrt(192)),
                         std=1.0)
    check_latent(c)


@pytest.mark.parametrize("bs", [8, 32, 64])
def test_latent_mfma_block_sizes(bs):
    rng = np.random.default_rng(bs)
    mb = 768 // bs
    past = rng.integers(100, 700, 3)
    c = make_latent_case(16, 576, 512, 3 * mb, bs, 3, dtype=BF16, seed=bs, new_lens=[1, 3, 1],
                         past=past, max_blocks=mb, do_rotary=1, rot_dim=64, rotary_offset=512,
                         scale=float(1 / np.sqrt(192)), std=1.0)
    check_latent(c)


@pytest.mark.parametrize("window,softcap,sink", [(100, 0.0, False), (-1, 30.0, True),
                                                 (37, 20.0, True)])
def test_latent_mfma_masks_softcap_sink(window, softcap, sink):
    c = make_latent_case(16, 576, 512, 3 * 48, 16, 3, dtype=BF16, seed=window + 3,
                         new_lens=[1, 9, 2], past=[600, 250, 0], max_blocks=48, do_rotary=1,
                         rot_dim=64, rotary_offset=512, scale=float(1 / np.sqrt(192)), std=1.0,
                         window=window, softcap=softcap,
                         head_sink=np.linspace(-1, 1, 16) if sink else None)
    check_latent(c)


def test_latent_mfma_long_context_splits():
    # contexts of ~6000 keys: split into chunks, partials merged by split_reduce_kernel
    c = make_latent_case(16, 576, 512, 2 * 400, 16, 2, dtype=BF16, seed=41, new_lens=[1, 1],
                         past=[6390, 5000], max_blocks=400, do_rotary=1, rot_dim=64,
                         rotary_offset=512, scale=float(1 / np.sqrt(192)), std=1.0)
    check_latent(c)


def test_latent_mfma_negative_scale():
    c = make_latent_case(16, 576, 512, 3 * 48, 16, 3, dtype=F16, seed=43, new_lens=[1, 4, 1],
                         past=[300, 20, 700], max_blocks=48, scale=-0.05, std=1.0)
    check_latent(c)


# 544 and 288: rows of an odd number of 64-dim pieces (the last direct load of each wavefront's
# share runs on half its lanes; the row's pieces past the last multiple of 8 stay unswizzled)
@pytest.mark.parametrize("d,vd", [(320, 256), (192, 128), (512, 512), (544, 512), (288, 256)])
def test_latent_mfma_value_sizes(d, vd):
    c = make_latent_case(32, d, vd, 3 * 48, 16, 3, dtype=BF16, seed=d + vd, new_lens=[1, 5, 2],
                         past=[500, 80, 3], max_blocks=48, do_rotary=1,
                         rot_dim=d - vd if d > vd else 64, rotary_offset=vd if d > vd else 0,
                         scale=float(1 / np.sqrt(d)), std=1.0)
    check_latent(c)
