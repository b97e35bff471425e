"""CPU tests of the C ABI: the library loads, exports every declared symbol, and the host
logic (claim predicate, metadata validation with the reference's "PagedAttention:" errors)
behaves like the reference -- all without launching device work."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import onnxruntime_ep_mlx_amd as ep
from onnxruntime_ep_mlx_amd import _capi as capi

ROOT = Path(__file__).resolve().parent.parent


def _declared_functions():
    text = (ROOT / "include" / "pa_mi355x.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    declared = _declared_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(capi.EXPORTS) == declared


def test_library_exports_only_declared_symbols():
    """The version script keeps every internal helper local: the dynamic symbol table holds the
    header's functions and nothing else of ours."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm is not available")
    out = subprocess.run([nm, "-D", "--defined-only", str(capi.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    names = {line.split()[-1] for line in out.splitlines() if line.split()[1:2] in (["T"], ["B"], ["D"])}
    ours = {n for n in names if not n.startswith("_")}
    assert ours == set(_declared_functions()), sorted(ours ^ set(_declared_functions()))


def test_version_and_error_channel():
    lib = capi.load()
    assert b"gfx950" in lib.pa_version()
    h = C.c_void_p()
    rc = lib.pa_pool_create(0, 16, 8, 128, capi.PA_DTYPE_BFLOAT16, C.byref(h))
    assert rc == capi.PA_ERR_INVALID_ARGUMENT
    assert b"invalid pool geometry" in lib.pa_last_error()


# ------------------------------------------------------------------------------ claim
def _node(dtype=capi.PA_DTYPE_BFLOAT16, H=32, KV=8, d=128, nb=40000, bs=16, T=64, B=64,
          mb=512, cache_dtype=None, rotary=True):
    n = capi.PaNodeInfo()
    cache_dtype = dtype if cache_dtype is None else cache_dtype
    n.num_inputs, n.num_outputs = 10 if rotary else 8, 1
    shapes = {0: [T, H * d], 1: [T, KV * d], 2: [T, KV * d], 3: [nb, bs, KV, d],
              4: [nb, bs, KV, d], 5: [B + 1], 6: [B], 7: [B, mb], 8: [8200, d // 2],
              9: [8200, d // 2]}
    dts = {0: dtype, 1: dtype, 2: dtype, 3: cache_dtype, 4: cache_dtype, 5: 10, 6: 10, 7: 10,
           8: dtype, 9: dtype}
    for i in range(n.num_inputs):
        n.input_present[i] = 1
        n.input_dtype[i] = dts[i]
        n.input_rank[i] = len(shapes[i])
        for j, s in enumerate(shapes[i]):
            n.input_shape[i][j] = s
    n.output_present[0] = 1
    n.output_dtype[0] = dtype
    n.output_rank[0] = 2
    n.output_shape[0][0], n.output_shape[0][1] = T, H * d
    n.num_heads, n.kv_num_heads = H, KV
    n.do_rotary = int(rotary)
    n.local_window_size = -1
    n.is_causal = 1
    return n


def _claim(n):
    buf = C.create_string_buffer(256)
    ok = capi.load().pa_paged_attention_claim(C.byref(n), buf, 256)
    return ok, buf.value.decode()


def test_claim_accepts_baseline_config3_node():
    assert _claim(_node()) == (1, "")


def test_claim_accepts_fp8_cache_with_block_scales():
    n = _node(cache_dtype=capi.PA_DTYPE_FP8_E4M3, rotary=False)
    n.num_inputs = 16
    for i in (14, 15):
        n.input_present[i] = 1
        n.input_dtype[i] = capi.PA_DTYPE_FLOAT32
        n.input_rank[i] = 2
        n.input_shape[i][0], n.input_shape[i][1] = 40000, 8
    assert _claim(n)[0] == 1
    n.input_shape[15][1] = 4
    assert "v_scale" in _claim(n)[1]


@pytest.mark.parametrize("mutate,reason", [
    (lambda n: setattr(n, "is_causal", 2), "is_causal must be 0 or 1"),
    (lambda n: n.output_dtype.__setitem__(0, capi.PA_DTYPE_FLOAT32),
     "only supported for fp16/bf16"),
    (lambda n: setattr(n, "kv_num_heads", 5), "positive multiple of kv_num_heads"),
    (lambda n: setattr(n, "local_window_size", 0), "local_window_size must be -1 or positive"),
    (lambda n: setattr(n, "softcap", -1.0), "softcap must be finite and non-negative"),
    (lambda n: (setattr(n, "rotary_offset", 4), n.input_shape[8].__setitem__(1, 32),
                n.input_shape[9].__setitem__(1, 32)), "rotary_offset must be a multiple of 8"),
    (lambda n: (n.input_shape[8].__setitem__(1, 80), n.input_shape[9].__setitem__(1, 80)),
     "must not exceed head_size"),
    (lambda n: n.input_shape[8].__setitem__(1, 80), "matching [positions,rotary_dim/2]"),
    (lambda n: setattr(n, "kv_cache_layout_latent", 1), "LATENT"),
    (lambda n: n.input_dtype.__setitem__(5, capi.PA_DTYPE_FLOAT32), "input 5 must be int32"),
    (lambda n: n.input_present.__setitem__(9, 0), "requires cos_cache and sin_cache"),
    (lambda n: n.input_dtype.__setitem__(4, capi.PA_INT8_DTYPE), "storage dtype"),
    (lambda n: n.input_dtype.__setitem__(3, capi.PA_INT8_DTYPE),
     "integer k cache requires PER_TENSOR or PER_CHANNEL"),
    (lambda n: setattr(n, "num_inputs", 18), "expects 8 required inputs"),
])
def test_claim_declines_with_reference_reasons(mutate, reason):
    n = _node()
    mutate(n)
    ok, why = _claim(n)
    assert ok == 0 and reason in why, why


def _int_node(bits=8, modes=(capi.PA_QUANT_PER_CHANNEL, capi.PA_QUANT_PER_CHANNEL), head=16,
              KV=2, H=4):
    """The reference's integer PagedAttention node (test_quantized_kv.py:344-392)."""
    width = head if bits == 8 else (head + 1) // 2
    storage = capi.PA_INT8_DTYPE if bits == 8 else capi.PA_UINT8_DTYPE
    n = _node(dtype=capi.PA_DTYPE_FLOAT16, H=H, KV=KV, d=head, nb=6, bs=4, T=3, B=3, mb=2,
              cache_dtype=storage, rotary=False)
    for i in (3, 4):
        n.input_shape[i][3] = width
    n.num_inputs = 16
    for side, i in enumerate((14, 15)):
        n.input_present[i] = 1
        n.input_dtype[i] = capi.PA_DTYPE_FLOAT32
        if modes[side] == capi.PA_QUANT_PER_TENSOR:
            n.input_rank[i] = 1
            n.input_shape[i][0] = 1
        else:
            n.input_rank[i] = 2
            n.input_shape[i][0], n.input_shape[i][1] = KV, head
    n.k_quant_type, n.v_quant_type = modes
    n.k_cache_dtype = n.v_cache_dtype = capi.PA_DTYPE_INT8 if bits == 8 else capi.PA_DTYPE_INT4
    return n


@pytest.mark.parametrize("bits,head", [(8, 16), (4, 16), (4, 7)])
@pytest.mark.parametrize("modes", [(1, 1), (2, 2), (1, 2)])
def test_claim_accepts_integer_caches(bits, head, modes):
    assert _claim(_int_node(bits, modes, head)) == (1, "")


def test_claim_int8_without_explicit_cache_dtype_and_packed_qkv():
    n = _int_node(8)
    n.k_cache_dtype = n.v_cache_dtype = 0  # int8 storage needs no explicit "int8"
    assert _claim(n)[0] == 1
    n = _node()
    n.input_present[1] = n.input_present[2] = 0  # packed [T, (H + 2 KV) * d] query
    n.input_shape[0][1] = (32 + 16) * 128
    assert _claim(n) == (1, "")


def _latent_node(d=16, vd=8, H=2):
    """test_paged_attention.py:727-744: LATENT node, kv 1, value and value_cache absent."""
    n = _node(dtype=capi.PA_DTYPE_FLOAT16, H=H, KV=1, d=d, nb=3, bs=4, T=2, B=1, mb=3,
              rotary=True)
    n.input_present[2] = n.input_present[4] = 0
    n.input_shape[8][1] = n.input_shape[9][1] = 4
    n.rotary_offset = 8
    n.v_head_size = vd
    n.has_scale_attr = 1
    n.kv_cache_layout_latent = 1
    n.output_shape[0][1] = H * vd
    return n


def test_claim_accepts_latent_layout():
    assert _claim(_latent_node()) == (1, "")


@pytest.mark.parametrize("mutate,reason", [
    (lambda n: setattr(n, "kv_num_heads", 2), "LATENT layout requires kv_num_heads=1"),
    (lambda n: n.input_present.__setitem__(4, 1), "requires absent value/value_cache"),
    (lambda n: setattr(n, "has_scale_attr", 0), "asymmetric value heads requires an explicit"),
    (lambda n: setattr(n, "v_head_size", 32), "v_head_size must not exceed head_size"),
    (lambda n: n.input_dtype.__setitem__(3, capi.PA_INT8_DTYPE),
     "quantized LATENT cache contract is not supported"),
    (lambda n: (setattr(n, "num_outputs", 3), n.output_present.__setitem__(2, 1)),
     "no separate value cache output"),
])
def test_claim_declines_broken_latent_nodes(mutate, reason):
    n = _latent_node()
    mutate(n)
    ok, why = _claim(n)
    assert ok == 0 and reason in why, why


# test_quantized_kv.py:615-641 (paged=True): each broken static contract is declined.
@pytest.mark.parametrize("bad,reason", [
    ("mode", "requires PER_TENSOR or PER_CHANNEL"),
    ("missing_scale", "requires a scale tensor"),
    ("scale_dtype", "k_scale must be float32"),
    ("scale_shape", "k_scale must contain 8 elements"),
    ("scale_last", "per-channel scales must end in head_size"),
    ("cache_dtype", "storage dtype"),
    ("output_dtype", "retain cache storage dtype"),
    ("packing", "uint8 requires explicit int4"),
    ("packing_absent", "uint8 requires explicit int4"),
])
def test_claim_declines_broken_integer_contracts(bad, reason):
    n = _int_node(4, head=4)
    if bad == "mode":
        n.k_quant_type = capi.PA_QUANT_NONE
    elif bad == "missing_scale":
        n.input_present[14] = 0
    elif bad == "scale_dtype":
        n.input_dtype[14] = capi.PA_DTYPE_FLOAT16
    elif bad == "scale_shape":
        n.input_shape[14][1] = 3
    elif bad == "scale_last":
        n.input_shape[14][0], n.input_shape[14][1] = 4, 2
    elif bad == "cache_dtype":
        n.input_dtype[4] = capi.PA_DTYPE_FLOAT16
    elif bad == "output_dtype":
        n.num_outputs = 2
        n.output_present[1] = 1
        n.output_dtype[1] = capi.PA_DTYPE_FLOAT16
    elif bad == "packing":
        n.k_cache_dtype = -1  # e.g. "float4e2m1"
    else:
        n.k_cache_dtype = 0
    ok, why = _claim(n)
    assert ok == 0 and reason in why, why


# ------------------------------------------------------------------------------ validation
def _io(cum, past, bt, slots=None, nb=8, bs=4, T=None, H=4, KV=2, d=8):
    """PagedAttention io with fake (never dereferenced) device pointers and real host copies:
    validation fails before any device work, so this runs without a GPU."""
    T = int(cum[-1]) if T is None else T
    keep = [np.ascontiguousarray(a, np.int32) for a in (cum, past, bt)]
    keep.append(None if slots is None else np.ascontiguousarray(slots, np.int32))
    fake = 0x1000
    cache = capi.PaCache(fake, fake, None, None, nb, bs, KV, d, capi.PA_DTYPE_FLOAT16)
    io = capi.PaIO(capi.PA_DTYPE_FLOAT16, T, H * d, fake, fake, fake, cache, fake, fake, fake,
                   len(cum) - 1, keep[2].shape[1], None, None, 0, 0,
                   fake if slots is not None else None, None, None, None,
                   keep[0].ctypes.data, keep[1].ctypes.data, keep[2].ctypes.data,
                   None if slots is None else keep[3].ctypes.data, fake)
    node = capi.PaNode(H, KV, 0.0, 0.0, -1, 0, 0, 0, 1, 1e-6)
    return node, io, keep


def _run_validation(node, io):
    lib = capi.load()
    rc = lib.pa_paged_attention(C.byref(node), C.byref(io), C.c_void_p(0x2000), 1 << 40, None)
    return rc, lib.pa_last_error().decode()


# test_attention_contracts.py:369-392
@pytest.mark.parametrize("invalid", ["cumulative", "negative_past", "too_long", "block", "slot"])
def test_invalid_live_metadata_errors(invalid):
    rng = np.random.default_rng(123)
    cum = np.array([0, 2, 3], np.int32)
    past = np.array([1, 2], np.int32)
    bt = rng.permutation(8).astype(np.int32).reshape(2, 4)
    slots = None
    if invalid == "cumulative":
        cum[1] = -1
    elif invalid == "negative_past":
        past[0] = -1
    elif invalid == "too_long":
        past[0] = 1000
    elif invalid == "block":
        bt.fill(-1)
    else:
        slots = np.full(3, 1000, np.int32)
    node, io, keep = _io(cum, past, bt, slots)
    rc, msg = _run_validation(node, io)
    assert rc == capi.PA_ERR_INVALID_ARGUMENT
    assert msg.startswith("PagedAttention:"), msg


def test_bad_head_counts_error():
    node, io, keep = _io(np.array([0, 1], np.int32), np.array([0], np.int32),
                         np.zeros((1, 2), np.int32))
    node.kv_num_heads = 3
    rc, msg = _run_validation(node, io)
    assert rc != 0 and msg == "PagedAttention: bad num_heads/kv_num_heads"


def test_workspace_query_is_pure_host():
    node, io, keep = _io(np.array([0, 1, 2], np.int32), np.array([100, 7], np.int32),
                         np.zeros((2, 4096), np.int32), nb=128, bs=4)
    n = capi.load().pa_paged_attention_workspace_bytes(C.byref(node), C.byref(io))
    assert n > 0 and n % 256 == 0


# GroupQueryAttention length rules (gqa_batched, attention.rs:614-631, :665-672): host-side
# checks that fail before any device work, so they run without a GPU
@pytest.mark.parametrize("seqlens,total,msg", [
    ([5, 9], 9, "invalid per-batch or maximum sequence lengths"),      # max != total - 1
    ([5, -1], 6, "invalid per-batch or maximum sequence lengths"),     # negative
    ([5, 40], 41, "exceeds available past cache"),                     # beyond capacity 32
])
def test_gqa_length_validation(seqlens, total, msg):
    from onnxruntime_ep_mlx_amd import _capi as capi
    lib = capi.load()
    host = np.asarray(seqlens, np.int32)
    node = capi.PaGqaNode(8, 2, 0.0, 0.0, -1, 0, 0, 1, 1e-6, 0)
    fake = 0x1000  # never dereferenced: validation fails first
    io = capi.PaGqaIO(dtype=capi.PA_DTYPE_BFLOAT16, batch=2, seq=1, query_hidden=8 * 64,
                      kv_seq=1, query=fake, key=fake, value=fake, past_key=fake,
                      past_value=fake + 64, past_capacity=32, present_key=fake,
                      present_value=fake + 64, seqlens_k=fake, host_seqlens_k=host.ctypes.data,
                      total_sequence_length=total, output=fake)
    nbytes = lib.pa_group_query_attention_workspace_bytes(C.byref(node), C.byref(io))
    assert nbytes > 0
    rc = lib.pa_group_query_attention(C.byref(node), C.byref(io), C.c_void_p(fake), nbytes, None)
    assert rc != 0
    err = lib.pa_last_error().decode()
    assert err.startswith("GroupQueryAttention:") and msg in err, err
