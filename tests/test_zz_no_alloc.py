"""pa_paged_attention_static (the allocation-free entry: its workspace is the library's per-GPU
static scratch) against pa_paged_attention with a caller workspace, through the C ABI.

Two calls in a row on the same scratch, the second with a smaller input: a planned prefill
(unit list, split flags and fp16 partials in the scratch) and then a small decode batch (balanced
split-K partials), plus a decode followed by an even smaller one.  Caches must be bit-identical to
the caller-workspace entry's; so must the decode outputs, which run the same kernels.  The
prefill's operand images (about 55 MB here) do not fit beside its partials in the scratch, so the
static entry runs that planned prefill with the in-loop value conversion: its output must agree
with the caller-workspace entry's within the parity bar (rel-L2 <= 2e-3).  A call whose workspace
exceeds the scratch even so is rejected on the host before any device work.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16
from pa_cases import make_case, run_gpu_op


def _prefill_case():
    rng = np.random.default_rng(1001)
    B, bs = 6, 16
    past = rng.integers(0, 3000, size=B)
    past[2] = 3900  # an item over the split threshold
    new = np.full(B, 512)
    mb = int((past.max() + 512 + bs - 1) // bs)
    return make_case(28, 4, 128, B * mb, bs, B, dtype=BF16, seed=1001, new_lens=new, past=past,
                     max_blocks=mb, std=1.0)


def _decode_case(B, seed):
    rng = np.random.default_rng(seed)
    bs = 16
    ctx = rng.integers(300, 3000, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    return make_case(32, 8, 128, B * mb, bs, B, dtype=BF16, seed=seed, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=mb, do_rotary=1, theta=500000.0, std=1.0)


def _same(case):
    a = run_gpu_op(case)
    b = run_gpu_op(case, static_scratch=True)
    for x, y, what in zip(a[1:], b[1:], ("key cache", "value cache")):
        assert np.array_equal(x, y), what
    dt = case["dtype"]
    if int(case["cum"][-1]) <= 64:
        assert np.array_equal(a[0], b[0]), "output"
    else:  # planned prefill: without operand images in the scratch
        err = orc.rel_l2(orc.decode(b[0], dt), orc.decode(a[0], dt))
        assert err <= 2e-3, err
    if int(case["cum"][-1]) <= 64:  # decode batches: the oracle too (the prefill one is slow)
        ref, ref_t, _, _ = orc.paged_attention_op(case)
        err = orc.rel_l2(orc.decode(b[0], case["dtype"]), orc.decode(ref_t, case["dtype"]))
        assert err <= 2e-3, err


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [("prefill", "decode16"), ("decode32", "decode5")])
def test_static_entry_matches_workspace_entry(first, second):
    cases = {"prefill": _prefill_case, "decode16": lambda: _decode_case(16, 17),
             "decode32": lambda: _decode_case(32, 33), "decode5": lambda: _decode_case(5, 6)}
    _same(cases[first]())
    _same(cases[second]())  # smaller input on the scratch the first call left behind


def test_static_entry_rejects_workspace_beyond_scratch():
    """Host-only: the size check precedes every device call (fake device pointers)."""
    from onnxruntime_ep_mlx_amd import _capi as capi
    lib = capi.load()
    H, KV, d, nb, bs = 64, 8, 128, 512, 16
    cum = np.array([0, 4096], np.int32)
    past = np.array([0], np.int32)
    bt = np.arange(nb, dtype=np.int32).reshape(1, nb)
    fake = 0x1000
    cache = capi.PaCache(fake, fake, None, None, nb, bs, KV, d, capi.PA_DTYPE_BFLOAT16)
    io = capi.PaIO(capi.PA_DTYPE_BFLOAT16, 4096, H * d, fake, fake, fake, cache, fake, fake,
                   fake, 1, nb, None, None, 0, 0, None, None, None, None, cum.ctypes.data,
                   past.ctypes.data, bt.ctypes.data, None, fake)
    node = capi.PaNode(H, KV, 0.0, 0.0, -1, 0, 0, 0, 1, 1e-6)
    need = lib.pa_paged_attention_workspace_bytes(C.byref(node), C.byref(io))
    assert need > capi.PA_STATIC_SCRATCH_BYTES
    rc = lib.pa_paged_attention_static(C.byref(node), C.byref(io), None)
    assert rc == capi.PA_ERR_UNSUPPORTED
    msg = lib.pa_last_error().decode()
    assert "static scratch" in msg, msg
    # the reported need is the call's without operand images (at most the full need), still
    # beyond the scratch
    import re
    got = int(re.search(r"needs (\d+) bytes", msg).group(1))
    assert capi.PA_STATIC_SCRATCH_BYTES < got <= need, msg
