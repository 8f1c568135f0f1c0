"""CPU-side checks of the C-ABI library: it loads, exports every entry point that
include/lgbm_hip.h declares, the ctypes struct layouts match the header, and
context creation without a GPU fails with a status (no abort)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from lightgbm_rs_amd import _abi
from lightgbm_rs_amd.backend import LIB_PATH, load_library

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lgbm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^int (lgbm_hip_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "build the library first (__graft_entry__.build())"
    lib = load_library()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), f"missing export {n}"


def test_struct_layouts_match_header():
    # Compile a tiny C program against the header and compare sizeof/offsetof.
    src = r"""
#include <stdio.h>
#include <stddef.h>
#include "lgbm_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu\n", sizeof(lgbm_gain_config), sizeof(lgbm_split_info),
         sizeof(lgbm_batched_feature), sizeof(lgbm_feature_meta), sizeof(lgbm_tree_out),
         sizeof(lgbm_layout_out), sizeof(lgbm_leaf_sums));
  printf("%zu %zu %zu %zu\n", offsetof(lgbm_gain_config, lambda_l2),
         offsetof(lgbm_split_info, gain), offsetof(lgbm_batched_feature, run_forward),
         offsetof(lgbm_tree_out, leaf_parent));
  return 0;
}
"""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "t.c")
        open(p, "w").write(src)
        exe = os.path.join(d, "t")
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), p, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    sizes = [int(x) for x in out[0].split()]
    offs = [int(x) for x in out[1].split()]
    assert sizes[:6] == [C.sizeof(_abi.GainConfig), C.sizeof(_abi.SplitInfo),
                         C.sizeof(_abi.BatchedFeature), C.sizeof(_abi.FeatureMeta),
                         C.sizeof(_abi.TreeOut), C.sizeof(_abi.LayoutOut)]
    assert offs == [_abi.GainConfig.lambda_l2.offset, _abi.SplitInfo.gain.offset,
                    _abi.BatchedFeature.run_forward.offset, _abi.TreeOut.leaf_parent.offset]


def test_status_codes_match_header():
    text = open(HEADER).read()
    codes = {int(v): k for k, v in re.findall(r"#define LGBM_HIP_(?:ERR_)?(\w+) \((-?\d+)\)", text)}
    codes[0] = "OK"
    for code in _abi.STATUS:
        assert code in codes


def test_create_without_device_returns_status():
    # In the build container there is no GPU: creation must fail cleanly.
    import torch  # noqa: F401  (only to mirror how callers load the runtime)
    if os.environ.get("LGBM_ASSUME_GPU"):
        pytest.skip("a GPU is present")
    lib = load_library()
    ctx = C.c_void_p()
    rc = lib.lgbm_hip_ctx_create(0, C.byref(ctx))
    if rc == 0:
        lib.lgbm_hip_ctx_destroy(ctx)
        pytest.skip("a HIP device is visible here")
    assert rc in (-3, -5, -6)
    buf = C.create_string_buffer(256)
    assert lib.lgbm_hip_last_error(None, buf, 256) == 0
    assert len(buf.value) > 0


def test_binary_boost_from_score_matches_oracle_and_capture():
    """The library's BinaryLogloss::boost_from_score against the oracle and the real
    binary's captured init score (-0.33647223662121273 = log(5/7) for the binary
    spine corpus, boosting/binary_gh_iterN.txt)."""
    import numpy as np

    from lightgbm_rs_amd import binary_boost_from_score
    from oracle import oracle
    y = np.array([0, 0, 0, 0, 0, 1, 0, 1, 1, 0, 1, 1], np.float32)
    assert binary_boost_from_score(y) == -0.33647223662121273
    rng = np.random.default_rng(4)
    for lab in [(rng.random(10001) < 0.3).astype(np.float32), np.ones(4, np.float32),
                np.zeros(4, np.float32), np.array([], np.float32)]:
        assert binary_boost_from_score(lab) == oracle.boost_from_score(lab)
    assert binary_boost_from_score(y, sigmoid=2.0) == -0.33647223662121273 / 2.0
