"""ctypes view of the C ABI (include/fa_mi355x.h, include/fa_probe.h).

This is the binding a non-torch host would use: plain pointers, sizes and a
hipStream_t as an integer. ``load()`` maps libfa_mi355x.so and declares every
exported signature; ``HEADER_SYMBOLS`` lists the functions the headers declare.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import re

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "libfa_mi355x.so"
INCLUDE = _HERE.parent / "include"

_vp, _i64, _i32p, _fp = C.c_void_p, C.c_int64, C.POINTER(C.c_int32), C.POINTER(C.c_float)

SIGNATURES = {
    "fa_status_str": (C.c_char_p, [C.c_int]),
    "fa_abi_version": (C.c_int, []),
    "fa_validate_fwd": (C.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64]),
    "fa_fwd_f16": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, C.c_int, _vp]),
    "fa_validate_decode": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _i64]),
    "fa_decode_workspace_floats": (_i64, [_i64, _i64, _i64, _i64]),
    "fa_decode_split_f16": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _vp, _vp, _vp]),
    "fa_lse_combine_f32": (C.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "fa_decode_paged_f16": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "fa_probe_mfma32": (C.c_int, [_vp, _vp, _vp, C.c_int, _vp]),
    "fa_probe_mfma16": (C.c_int, [_vp, _vp, _vp, C.c_int, _vp]),
    "fa_probe_tr16_raw": (C.c_int, [_vp, _vp, _vp]),
    "fa_probe_permlane": (C.c_int, [_vp, _vp, _vp]),
    "fa_probe_frags": (C.c_int, [_vp, _vp, _vp, _i64, _vp]),
    "fa_probe_chain": (C.c_int, [_vp, _vp, _vp, _vp, _i64, _vp]),
    "fa_validate_bwd": (C.c_int, [_vp] * 10 + [_i64] * 4),
    "fa_bwd_workspace_floats": (_i64, [_i64, _i64, _i64]),
    "fa_bwd_f16": (C.c_int, [_vp] * 10 + [_i64] * 4 + [C.c_int, _vp]),
    "fa_validate_fwd_gqa": (C.c_int, [_vp] * 4 + [_i64] * 5),
    "fa_fwd_gqa_f16": (C.c_int, [_vp] * 5 + [_i64] * 5 + [C.c_int, _vp]),
    "fa_fwd_bf16": (C.c_int, [_vp] * 5 + [_i64] * 5 + [C.c_int, _vp]),
    "fa_validate_fwd_varlen": (C.c_int, [_vp] * 5 + [_i64] * 6),
    "fa_fwd_varlen_f16": (C.c_int, [_vp] * 6 + [_i64] * 6 + [C.c_int, _vp]),
    "fa_decode_paged_gqa_f16": (C.c_int, [_vp] * 5 + [_i64] * 8 + [_vp] * 5),
    "fa_decode_paged_bf16": (C.c_int, [_vp] * 5 + [_i64] * 8 + [_vp] * 5),
    "fa_decode_paged_noalloc_f16": (C.c_int, [_vp] * 5 + [_i64] * 8 + [_vp] * 3),
    "fa_validate_kv_append": (C.c_int, [_vp] * 8 + [_i64] * 7),
    "fa_kv_append_f16": (C.c_int, [_vp] * 8 + [_i64] * 7 + [_vp]),
    "fa_kv_append_bf16": (C.c_int, [_vp] * 8 + [_i64] * 7 + [_vp]),
    "fa_bwd_gqa_workspace_floats": (_i64, [_i64] * 5),
    "fa_bwd_gqa_f16": (C.c_int, [_vp] * 10 + [_i64] * 5 + [C.c_int, _vp]),
    "fa_bwd_bf16": (C.c_int, [_vp] * 10 + [_i64] * 5 + [C.c_int, _vp]),
    "fa_fwd_splitkv_plan": (C.c_int, [_i64] * 4 + [C.c_int]),
    "fa_fwd_splitkv_workspace_floats": (_i64, [_i64] * 5),
    "fa_fwd_splitkv_f16": (C.c_int, [_vp] * 6 + [_i64] * 5 + [C.c_int, _i64, _vp]),
    "fa_bwd_varlen_f16": (C.c_int, [_vp] * 11 + [_i64] * 6 + [C.c_int, _vp]),
    "fa_validate_bwd_varlen": (C.c_int, [_vp] * 11 + [_i64] * 6),
    "fa_probe_fwd_variant": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, C.c_int, C.c_int, _vp]),
    "fa_probe_fwd_variants": (C.c_int, [_vp, C.c_int, _i64, C.c_int]),
    "fa_probe_default_variant": (C.c_int, [_i64]),
    "fa_probe_choose_variant": (C.c_int, [_i64, C.c_int, _i64, _i64, C.c_int]),
    "fa_probe_splitkv_plan_cus": (C.c_int, [_i64] * 4 + [C.c_int, C.c_int]),
    "fa_probe_read_bw": (C.c_int, [_vp, _i64, C.c_int, _vp, _vp]),
    "fa_probe_gather_bw": (C.c_int, [_vp, _vp, _vp, _i64, C.c_int, C.c_int, _vp, _vp]),
}

DECODE_SCRATCH_FLOATS = 1 << 22   # FA_DECODE_SCRATCH_FLOATS

STATUS = {
    "FA_OK": 0, "FA_ERR_NULL_POINTER": 1, "FA_ERR_HEAD_DIM": 2, "FA_ERR_SEQ_LEN": 3,
    "FA_ERR_BATCH_HEADS": 4, "FA_ERR_ALIGNMENT": 5, "FA_ERR_TOO_LARGE": 6,
    "FA_ERR_PAGE_SIZE": 7, "FA_ERR_NUM_SPLITS": 8, "FA_ERR_MAX_PAGES": 9,
    "FA_ERR_NUM_PAGES": 10, "FA_ERR_KV_HEADS": 11, "FA_ERR_SCRATCH_SIZE": 12,
}


def header_symbols() -> list[str]:
    """Function names declared in include/*.h."""
    names = []
    for h in sorted(INCLUDE.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(fa_[a-z0-9_]+)\s*\(", text):
            if m.group(1) not in names:
                names.append(m.group(1))
    return names


def load(path: pathlib.Path | str = LIB_PATH) -> C.CDLL:
    """Map the library and declare argument/return types of every C-ABI function."""
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
