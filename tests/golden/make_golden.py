"""Writes the committed golden fixtures of the paged-attention path (tests/golden/*.npz).

Each fixture holds one seeded case (the inputs exactly as uploaded: raw dtype bits) and the CPU
oracle's results for it: the key/value pools after the append (bit patterns), the output rounded
to the activation dtype (bit patterns) and the float64 output.  The oracle is itself pinned by
tests/test_oracle.py (torch/numpy converters, closed forms, brute force, the reference's
known answers); the fixtures freeze its results so that tests/test_golden.py catches any drift
and tests/test_gpu_golden.py checks the HIP path against stored numbers.

    python tests/golden/make_golden.py          # rewrites every fixture
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import _oracle as orc  # noqa: E402
from _oracle import BF16, E4M3, F16  # noqa: E402
from pa_cases import make_case  # noqa: E402

SCALARS = ("num_heads", "kv_num_heads", "head_dim", "dtype", "cache_dtype", "softcap",
           "local_window_size", "is_causal", "scale", "rotary_offset", "rotary_interleaved",
           "qk_norm_epsilon")


def cases() -> dict:
    """Small geometries covering the path's forms (decode MFMA, prefill, fp8 pages, rotary,
    sink/softcap/window, slot mapping); every fixture stays well under 100 KB."""
    return {
        # decode, bf16, RoPE theta 500000 (BASELINE.json config 3 form), balanced MFMA path
        "decode_bf16_rope": make_case(8, 2, 64, 9, 16, 3, dtype=BF16, seed=101,
                                      new_lens=[1, 1, 1], past=[5, 20, 40], max_blocks=3,
                                      do_rotary=1, theta=500000.0, std=1.0),
        # prefill chunk, fp16, causal inside the chunk, two sequences
        "prefill_f16_causal": make_case(4, 2, 64, 4, 16, 2, dtype=F16, seed=102,
                                        new_lens=[5, 3], past=[7, 0], max_blocks=2),
        # fp8 e4m3 pages with per-(block, kv-head) scales (config 5 form), bf16 activations
        "decode_fp8": make_case(8, 2, 128, 4, 16, 2, dtype=BF16, cache_dtype=E4M3, seed=103,
                                new_lens=[1, 1], past=[30, 12], max_blocks=2, std=1.0),
        # attributes: sink + softcap + local window, interleaved rotary with an offset
        "decode_f16_attrs": make_case(4, 1, 64, 6, 16, 2, dtype=F16, seed=104, new_lens=[2, 1],
                                      past=[33, 9], max_blocks=3, do_rotary=1, interleaved=1,
                                      rot_dim=32, rotary_offset=16,
                                      head_sink=[0.5, -1.0, 0.25, 2.0], softcap=20.0, window=24),
        # explicit slot mapping (block size 4, the reference's test geometry)
        "slot_mapping_f16": make_case(2, 1, 16, 8, 4, 2, dtype=F16, seed=105, new_lens=[2, 1],
                                      past=[3, 6], max_blocks=4,
                                      slot_mapping=[13, 14, 30]),
    }


def save(name: str, case: dict) -> Path:
    ref, ref_t, kc, vc = orc.paged_attention_op(case)
    arrays = {f"in_{k}": np.asarray(v) for k, v in case.items()
              if isinstance(v, np.ndarray)}
    arrays.update({f"attr_{k}": np.asarray(case[k]) for k in SCALARS if k in case})
    arrays.update(exp_output_f64=ref, exp_output_t=ref_t, exp_key_cache=kc, exp_value_cache=vc)
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, **arrays)
    return path


def load(path: Path):
    """Return (case dict, expected dict) from a fixture file (no pickles)."""
    z = np.load(path, allow_pickle=False)
    case, exp = {}, {}
    for k in z.files:
        if k.startswith("in_"):
            case[k[3:]] = z[k]
        elif k.startswith("attr_"):
            v = z[k]
            case[k[5:]] = v.item()
        elif k.startswith("exp_"):
            exp[k[4:]] = z[k]
    return case, exp


if __name__ == "__main__":
    for n, c in cases().items():
        p = save(n, c)
        print(f"{p.name}: {p.stat().st_size} bytes")
