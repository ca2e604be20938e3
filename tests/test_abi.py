"""The C-ABI library loads without a GPU, exports every entry point include/*.h declares, and its host-side
argument checks reject bad shapes before any launch (CPU only: no kernel runs here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared_functions():
    src = "\n".join(open(h).read() for h in HEADERS)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(smel_\w+)\s*\(", src, flags=re.M)))


def test_header_parses():
    names = declared_functions()
    assert "smel_gmm_fwd" in names and "smel_route" in names and len(names) >= 15


def test_library_exports_every_declared_symbol():
    from smel import _lib
    L = _lib.load()
    for n in declared_functions():
        assert hasattr(L, n), n
    # the Python binding types every declared symbol, and nothing undeclared
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_wset_layout_matches_header():
    from smel import _lib
    # 7 pointers, two int64, two int32
    assert ctypes.sizeof(_lib.WSet) == 7 * 8 + 2 * 8 + 2 * 4


PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "smel_moe.h"
#include "smel_f32.h"
#define F(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main() {
  printf("smel_wset %zu\nsmel_wg_dest %zu\nsmel_wg_job %zu\nsmel_lora_set %zu\n", sizeof(smel_wset),
         sizeof(smel_wg_dest), sizeof(smel_wg_job), sizeof(smel_lora_set));
  F(smel_wset, R) F(smel_wset, group) F(smel_wset, flags) F(smel_wg_dest, s_idx) F(smel_wg_dest, p0) F(smel_wg_dest, nq)
  F(smel_wg_job, ldr) F(smel_wg_job, r_gather) F(smel_wg_job, Q) F(smel_wg_job, ldl) F(smel_wg_job, dest)
  F(smel_lora_set, n) F(smel_lora_set, r) F(smel_lora_set, fwd_gu) F(smel_lora_set, at_dn)
  printf("smel_fwd_lora_rows %zu\nsmel_bwd_lora_rows %zu\n", sizeof(smel_fwd_lora_rows), sizeof(smel_bwd_lora_rows));
  F(smel_fwd_lora_rows, scale_sh) F(smel_fwd_lora_rows, part) F(smel_fwd_lora_rows, parts) F(smel_fwd_lora_rows, ext_out)
  F(smel_bwd_lora_rows, scale_sh) F(smel_bwd_lora_rows, n_sel) F(smel_bwd_lora_rows, planes) F(smel_bwd_lora_rows, part)
  F(smel_bwd_lora_rows, parts)
  printf("smel_wset_f32 %zu\n", sizeof(smel_wset_f32));
  F(smel_wset_f32, wsh) F(smel_wset_f32, R) F(smel_wset_f32, C) F(smel_wset_f32, group) F(smel_wset_f32, kinds)
  F(smel_wset_f32, q4_round_bf16)
  return 0;
}
"""


def test_struct_layouts_match_header(tmp_path):
    """The ctypes mirrors of the header's structs have the C compiler's sizes and field offsets."""
    import shutil
    import subprocess
    from smel import _lib
    cxx = shutil.which("g++")
    if cxx is None or not os.path.exists("/opt/rocm/include/hip/hip_runtime.h"):
        pytest.skip("no host compiler / HIP headers")
    src = tmp_path / "probe.cpp"
    src.write_text(PROBE)
    exe = tmp_path / "probe"
    subprocess.run([cxx, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"),
                    str(src), "-o", str(exe)], check=True, capture_output=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    mirror = {"smel_wset": _lib.WSet, "smel_wg_dest": _lib.WgDest, "smel_wg_job": _lib.WgJob,
              "smel_lora_set": _lib.LoraSet, "smel_fwd_lora_rows": _lib.FwdLoraRows,
              "smel_bwd_lora_rows": _lib.BwdLoraRows, "smel_wset_f32": _lib.WSetF32}
    for key, val in got.items():
        if "." in key:
            t, f = key.split(".")
            assert getattr(mirror[t], f).offset == int(val), key
        else:
            assert ctypes.sizeof(mirror[key]) == int(val), key


def test_host_side_rejections():
    """Shape checks happen on the host, before any launch, so they are safe without a GPU."""
    from smel import _lib
    L = _lib.load()
    assert L.smel_dispatch_max_tiles(32736, 256, 4092, 128) == (32736 + 127) // 128 + 256 + 32 + 1
    assert L.smel_dispatch_ws_size(32736, 256) == 32 * 256 + 32 and L.smel_dispatch_ws_size(0, 8) == 0
    # dispatch: a merged tile list needs 128 < merge_rows <= 192, its outputs and the group kinds
    d = (16, 0, 4, 2, 8, 0, 128)
    for mr, gk, tm in ((200, 16, 16), (160, None, 16), (160, 16, None), (100, 16, 16)):
        assert L.smel_dispatch(*d, gk, 16, 16, 16, 16, 16, 16, 16, 16, mr, tm, 16, 16, None) == -1
        assert b"merged tile list" in L.smel_last_error()
    # gmm_fwd: the merged list on an int4 bank without the fast dequant form, or with K not a multiple of 64
    wm = _lib.WSet()
    wm.R, wm.C, wm.group, wm.q4, wm.sz4, wm.flags = 1024, 2048, 64, 16, 16, _lib.WSET_MERGED_LIST
    for epi, flags, C in ((1, _lib.WSET_MERGED_LIST, 2048), (0, _lib.WSET_MERGED_LIST, 2048),
                          (0, _lib.WSET_MERGED_LIST | _lib.WSET_FAST_DQ, 2016)):
        wm.flags, wm.C, wm.group = flags, C, 32 if C % 64 else 64
        assert L.smel_gmm_fwd(ctypes.byref(wm), None, 16, 16, 1, 16, 2048, 4, 0, None, 0, 1, None, epi, 0, 16, 1024,
                              16, None) == -1
        assert b"merged tile list" in L.smel_last_error()
    # route: too many experts
    rc = L.smel_route(1, 1, None, 4, 64, 600, 8, 1, 1, None, 1, 1, None, 1, None)
    assert rc == -2 and b"E=600" in L.smel_last_error()
    # route: hidden not a multiple of 64
    assert L.smel_route(1, 1, None, 4, 96, 8, 2, 1, 1, None, 1, 1, None, 1, None) == -2
    assert L.smel_route_ld(256, 1) == 288 and L.smel_route_ld(250, 0) == 256
    # dequant: K not a multiple of the group
    assert L.smel_dequant_int4(1, 1, 1, 1, 4, 96, 64, 0, None) == -1
    # gmm: null weight set
    assert L.smel_gmm_fwd(None, 1, 1, 1, 1, 1, 64, 4, 0, None, 0, 1, None, 0, 0, 1, 64, None, None) == -1
    w = _lib.WSet()
    w.R, w.C, w.group = 64, 48, 64
    assert L.smel_gmm_fwd(ctypes.byref(w), 1, 1, 1, 1, 16, 48, 4, 0, None, 0, 1, None, 0, 0, 16, 64, None, None) == -2
    # packing: sizes and rejections
    assert L.smel_packed_bytes(_lib.PACK_Q4, 64, 2048) == 2 * 32 * 1024
    assert L.smel_packed_bytes(_lib.PACK_SZ, 64, 2048) == 2 * 8 * 1024
    assert L.smel_packed_bytes(_lib.PACK_BF16, 33, 96) == 2 * 2 * 4096
    assert L.smel_packed_bytes(7, 64, 64) == -1
    assert L.smel_pack_int4(1, 1, 1, 64, 96, 64, 1, 1, None) == -2      # group does not divide K
    assert L.smel_pack_bf16(1, 64, 60, 64, 1, None) == -2               # K not a multiple of 8
    # LoRA layouts: rank above 16 with one gate_up plane, above 32 with two, a third plane
    for r, planes in ((17, 1), (33, 2), (8, 3)):
        with pytest.raises(_lib.SmelError):
            _lib.call("smel_lora_prep", None, None, None, None, None, None, 2, r, planes, 64, 64, None, None, None,
                      None, None, None, None, None, None)
    with pytest.raises(_lib.SmelError):   # ext row stride other than one or two planes
        _lib.call("smel_lora_ext", 8, 8, 1, None, 16, 64, 4, 0, None, 0, 1, None, 16, 64, 1.0, 1.0, 16, 48, None)
    # LoRA weight gradients: an L row stride other than 32 / 64, and a destination outside the 32 x Q result, are
    # rejected on the host
    jobs = (_lib.WgJob * 4)()
    jobs[0].L, jobs[0].Rm, jobs[0].ldr, jobs[0].r_rows, jobs[0].Q, jobs[0].ldl = 8, 16, 64, 4, 64, 48
    assert L.smel_lora_wgrad(jobs, 1, 1, 1, 0, 1, 0, 4, 0, 1, None, None, None, 4, 1, 1 << 20, None) == -1
    assert b"stride" in L.smel_last_error()
    jobs[0].ldl = 64
    jobs[0].dest[1][0].ptr, jobs[0].dest[1][0].p0, jobs[0].dest[1][0].np, jobs[0].dest[1][0].nq = 16, 20, 16, 64
    assert L.smel_lora_wgrad_ws_floats(jobs, 1, 1, 4) == 1 * (1 + 1) * 32 * 128
    assert L.smel_lora_wgrad(jobs, 1, 1, 1, 0, 1, 0, 4, 0, 1, None, None, None, 4, 1, 1 << 20, None) == -1
    assert b"destination" in L.smel_last_error()
    jobs[0].dest[1][0].ptr = None
    assert L.smel_lora_wgrad(jobs, 1, 1, 1, 0, 1, 0, 4, 0, 1, None, None, None, 4, 1, 16, None) == -1
    assert b"workspace" in L.smel_last_error()
    # transposed layouts (backward GEMM operand): sizes and rejections
    assert L.smel_packed_t_bytes(_lib.PACK_Q4, 2, 1024, 2048, 64) == 2 * 64 * 16 * 1024
    assert L.smel_packed_t_bytes(_lib.PACK_SZ, 2, 1024, 2048, 64) == 2 * 32 * 16 * 512
    assert L.smel_packed_t_bytes(_lib.PACK_BF16, 1, 288, 2048, 0) == 64 * 5 * 4096
    assert L.smel_packed_t_bytes(_lib.PACK_SZ, 1, 64, 96, 64) == -1      # group does not divide C
    assert L.smel_pack_int4_t(1, 1, 1, 1, 64, 96, 64, 0, 1, 1, None) == -2  # group does not divide C
    assert L.smel_pack_int4_t(1, 1, 1, 1, 64, 128, 64, 2, 16, 16, None) == -1   # fast is 0 or 1
    assert L.smel_int4_fast_ok(None, None, 4, None, None) == -1
    assert L.smel_pack_bf16_t(1, 1, 64, 48, 64, 1, None) == -2           # C not a multiple of 32
    # LoRA rows from GEMM epilogues: partial count other than the producing GEMM's column blocks, ext given beside the
    # partials, a third plane
    w = _lib.WSet()
    w.R, w.C = 2048, 512
    lr = _lib.BwdLoraRows(None, 16, 1.0, 1.0, 0, 1, 16, 3)
    args = (ctypes.byref(w), None, 16, 16, 1, 16, 2048, 4, 0, None, 0, 1, None)
    assert L.smel_gmm_bwd_lr(*args, 1, 0, 16, 16, 16, 16, 1024, 16, ctypes.byref(lr), None) == -1
    assert b"partials" in L.smel_last_error()
    lr.parts = L.smel_gmm_bwd_nblocks(512)
    w.R, w.C = 512, 2048
    assert L.smel_gmm_bwd_lr(ctypes.byref(w), None, 16, 16, 1, 16, 1024, 4, 0, None, 0, 1, 16, 0, 0, None, None, None,
                             16, 2048, None, ctypes.byref(lr), None) == -1   # ext and partials together
    assert L.smel_lora_rows_sum(16, 16, 4, None, 1, 1, 16, 2, 3, 16, None) == -1
    fl = _lib.FwdLoraRows(None, 16, 1.0, 1.0, 16, 3, None)
    w.R, w.C = 1024, 2048
    assert L.smel_gmm_fwd_lr(ctypes.byref(w), None, 16, 16, 1, 16, 2048, 4, 0, None, 0, 1, None, 1, 0, 16, 512, None,
                             ctypes.byref(fl), None) == -1   # 3 partials for the gate_up forward's 4 column blocks


def test_f32_host_side_rejections():
    """The fp32 path's entry points check their arguments on the host before any launch."""
    from smel import _lib
    L = _lib.load()
    w = _lib.WSetF32()
    w.R, w.C, w.kinds = 64, 128, 1 << _lib.KIND_SHARED
    ok = (ctypes.byref(w), 0, None, 16, 16, 1, 16, 128, 1.0, 0.0, 16, 64, None)
    assert L.smel_gmm_f32(*ok) == -1 and b"shared" in L.smel_last_error()        # no shared weights
    w.wsh = 16
    assert L.smel_gmm_f32(ctypes.byref(w), 0, None, 16, 16, 1, 16, 128, 1.0, 0.5, 16, 64, None) == -1   # beta
    assert L.smel_gmm_f32(ctypes.byref(w), 2, None, 16, 16, 1, 16, 128, 1.0, 0.0, 16, 64, None) == -1   # trans
    assert L.smel_gmm_f32(ctypes.byref(w), 0, None, 16, 16, 1, 16, 64, 1.0, 0.0, 16, 64, None) == -1    # lda < K
    assert L.smel_gmm_f32(ctypes.byref(w), 1, None, 16, 16, 1, 16, 64, 1.0, 0.0, 16, 64, None) == -1    # ldc < N
    w.kinds = 1 << _lib.KIND_INT4
    assert L.smel_gmm_f32(ctypes.byref(w), 0, None, 16, 16, 1, 16, 128, 1.0, 0.0, 16, 64, None) == -1   # no q4
    w.q4 = w.scale = w.zero = 16
    w.group = 48                                                                                        # !| C
    assert L.smel_gmm_f32(ctypes.byref(w), 0, None, 16, 16, 1, 16, 128, 1.0, 0.0, 16, 64, None) == -1
    w.kinds = 1 << 5
    assert L.smel_gmm_f32(ctypes.byref(w), 0, None, 16, 16, 1, 16, 128, 1.0, 0.0, 16, 64, None) == -1   # kinds
    assert L.smel_wgrad_f32(16, 8, 16, 64, 16, 16, 1, 16, 64, 1.0, 16, 1024, None) == -1   # ldx < M
    assert L.smel_wgrad_f32(16, 16, 16, 64, 16, 16, 1, 16, 64, 1.0, 16, 512, None) == -1   # c_stride < M N
    assert L.smel_route_select_f32(16, 600, 4, 600, 8, None, 16, 16, 16, 16, None) == -2
    assert L.smel_route_select_f32(16, 64, 4, 64, 17, None, 16, 16, 16, 16, None) == -2
    assert L.smel_act_gate_f32(16, 64, 4, 64, 2, 16, 64, None) == -1                       # act id
    assert L.smel_act_gate_f32(16, 100, 4, 64, 0, 16, 64, None) == -1                      # ldh < 2I
    assert L.smel_combine_f32(16, 16, 16, 4, 65, 64, 16, None) == -1                       # K > 64


def test_product_path_does_not_reach_the_oracle():
    """Nothing under smel-ft_amd/ imports the oracle or the reference."""
    pkg = os.path.join(ROOT, "smel-ft_amd")
    for dp, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                s = open(os.path.join(dp, f)).read()
                assert "oracle" not in s.replace("Oracle", ""), f
                assert "/root/reference" not in s, f
