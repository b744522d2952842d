"""The C-ABI library loads, exports every entry point include/pkv.h declares,
and rejects bad arguments before launching anything. CPU only: no call here
reaches a kernel."""
import os
import re

import pkv

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pkv.h")


def declared():
    text = open(HDR).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(pkv._lib, n), n
    assert set(names) <= set(pkv.exported_symbols())


def test_status_strings():
    assert pkv.strerror(0) == "ok"
    assert pkv.strerror(pkv.ERR_UNSUPPORTED) == "unsupported shape"
    assert pkv.version() >= 1


def test_invalid_and_unsupported_arguments_return_before_launch():
    L = pkv._lib
    # decode: G = Hq / Hkv outside 1, 2, 4, 6, 8 (or Hq not a multiple of
    # Hkv) is unsupported, block size must be 16, for the fused step too
    for Hq, Hkv in ((10, 2), (12, 8), (3, 2), (24, 2)):
        assert L.pkv_attn_decode(1, 1, 1, 1, 8192, Hq, Hkv, 1, 1, 1, 4, 16, 1, 0.1, 1, 0, None, 1, 3, 10, 1,
                                 1 << 30, None) == pkv.ERR_UNSUPPORTED
    assert L.pkv_attn_decode_step(16, 16, 4096, 16, 16, 16, 16, 16, 12288, 10, 2, 16, 16, 16, 4, 16, 16, 0.1, 16, 0,
                                  None, 1, 3, 10, 256, 1 << 30, None) == pkv.ERR_UNSUPPORTED
    assert L.pkv_attn_decode(1, 1, 1, 1, 8192, 16, 4, 1, 1, 1, 4, 32, 1, 0.1, 1, 0, None, 1, 3, 10, 1, 1 << 30,
                             None) == pkv.ERR_UNSUPPORTED
    # null pointers, short workspace, misaligned pointers
    assert L.pkv_attn_decode(None, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, 16, 0, None, 1, 3, 10, 256,
                             1 << 30, None) == pkv.ERR_INVALID
    assert L.pkv_attn_decode(16, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, 16, 0, None, 1, 3, 10, 256,
                             16, None) == pkv.ERR_INVALID
    assert L.pkv_attn_decode(18, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, 16, 0, None, 1, 3, 10, 256,
                             1 << 30, None) == pkv.ERR_INVALID
    # E4M3 decode / verify: scales required; verify needs cu; no fused append
    for fn in (L.pkv_attn_decode_e4m3, L.pkv_attn_verify_e4m3):
        assert fn(16, 16, 16, None, None, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, 16, 0, None, 1, 3, 10, 256,
                  1 << 30, None) == pkv.ERR_INVALID
    assert L.pkv_attn_verify_e4m3(16, 16, 16, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, None, 0, None, 1,
                                  3, 10, 256, 1 << 30, None) == pkv.ERR_INVALID
    assert L.pkv_attn_decode_e4m3(16, 16, 16, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, None, 0, None, 1,
                                  3, 10, 256, 16, None) == pkv.ERR_INVALID  # short workspace
    # zero tokens is a no-op
    assert L.pkv_attn_decode(None, None, None, None, 10240, 16, 4, None, None, None, 4, 16, None, 0.1, None, 0, None,
                             1, 0, 10, None, 0, None) == pkv.OK
    assert L.pkv_append(1, 1, 16, 1, -1, 4, 512, 1, 1, 10, None) == pkv.ERR_INVALID
    assert L.pkv_append(1, 1, 100, 1, 4, 4, 512, 1, 1, 10, None) == pkv.ERR_INVALID  # stride < row
    assert L.pkv_append(None, None, 0, None, 0, 4, 512, None, None, 10, None) == pkv.OK
    assert L.pkv_page_copy(16, 16, 16, 16, 1, 100, 10, None) == pkv.ERR_INVALID  # page bytes % 16
    assert L.pkv_gather(16, 16, 16, -1, 16, 4, 512, 10, 16, 16, None) == pkv.ERR_INVALID
    assert L.pkv_attn_decode_config(0, 32) == pkv.ERR_INVALID
    assert L.pkv_mtp_next(16, 16, 16, 4, 16, 0, 16, 16, 1, 16, 16, 16, 2, None) == pkv.ERR_INVALID  # max_blocks
    assert L.pkv_mtp_next(None, 16, 16, 4, 16, 4, 16, 16, 1, 16, 16, 16, 2, None) == pkv.ERR_INVALID
    assert L.pkv_mtp_next(None, None, None, 0, None, 4, 16, None, 1, None, None, None, 0, None) == pkv.OK


def test_workspace_grows_with_tokens():
    a, b = pkv.attn_decode_workspace(1, 16), pkv.attn_decode_workspace(64, 16)
    assert b > a > 0
    assert (b - a) >= 63 * 16 * 256 * 4


def test_reference_abi_code_object_exports_the_reference_kernel_names(tmp_path):
    """pkv_kernels.hsaco (a bundle for hipModuleLoadData) holds the gfx950
    code object whose kernel symbols are the reference engine's names
    (src/model.rs:1053-1061, fa_shape :58-79)."""
    import subprocess
    from pkv import refabi
    bundler = "/opt/rocm/llvm/bin/clang-offload-bundler"
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    co = tmp_path / "gfx950.co"
    subprocess.run([bundler, "--unbundle", "--type=o", f"--input={refabi.HSACO}", f"--output={co}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950"], check=True)
    syms = subprocess.run([readelf, "--syms", "--wide", str(co)], check=True, capture_output=True, text=True).stdout
    kernels = {line.split()[-1] for line in syms.splitlines() if " FUNC " in line and "GLOBAL" in line}
    names = ["attn_prep", "attn_merge", "attn_groupr_g4_t2_k32", "attn_mfma_g4_t2", "mtp_next"]
    # decode for every group the reference instantiates (qwen35.cu:1330-1334)
    names += [f"attn_paged{e}_g{g}" for e in ("", "8") for g in (1, 2, 4, 6, 8)]
    # the prompt kernel gfx950's fa_shape picks for each group and cache type
    names += [refabi.flash_launch(100, 3, 4, g=g, fp8=f8)[0] for g in (1, 2, 4, 6, 8) for f8 in (False, True)]
    for name in names:
        assert name in kernels, (name, sorted(kernels)[:20])


def test_fp8_next_validates_and_clears():
    """pkv_attn_fp8_next: mode 0 / 1 / 2 only; a copy request needs both
    buffers and a row capacity; mode 0 clears (host only, nothing launched)."""
    L = pkv._lib
    assert L.pkv_attn_fp8_next(None, None, 3, 10) == pkv.ERR_INVALID
    assert L.pkv_attn_fp8_next(16, None, 1, 10) == pkv.ERR_INVALID
    assert L.pkv_attn_fp8_next(16, 16, 2, 0) == pkv.ERR_INVALID
    assert L.pkv_attn_fp8_next(16, 16, 1, 10) == pkv.OK
    # a decode call with T > frows is refused before any launch
    assert L.pkv_attn_decode(16, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16, 0.1, 16, 0, None, 1, 11, 10, 256,
                             1 << 30, None) == pkv.ERR_INVALID
    assert L.pkv_attn_fp8_next(None, None, 0, 0) == pkv.OK


def test_reference_launch_shapes():
    """The restated host formulas the code object is launched with."""
    from pkv import refabi
    assert refabi.split_ranges(64, 4, 256) == 4       # config 3 on 256 CUs
    assert refabi.split_ranges(1, 4, 256) == 64       # config 2: SPLIT_MAX
    assert refabi.split_ranges(300, 4, 256) == 1
    name, grid, threads, smem = refabi.flash_launch(100, 3, 4)
    assert (name, grid, threads, smem) == ("attn_groupr_g4_t2_k32", (7, 4, 1), 256, 67584)
    name, grid, threads, smem = refabi.flash_launch(100, 3, 4, mfma=True)
    assert (name, grid, threads, smem) == ("attn_mfma_g4_t2", (7, 4, 1), 512, 37376)
    name, grid, threads, smem = refabi.flash_launch(100, 3, 4, fp8=True)
    assert (name, grid, threads, smem) == ("attn_group8_g4_t2_k16", (7, 4, 1), 256, 101376)
    # other groups (fa_shape arm (_, 6, false) and the 16-key default)
    assert refabi.flash_launch(100, 3, 4, g=6) == ("attn_groupr_g6_t1_k32", (10, 4, 1), 192, 67584)
    assert refabi.flash_launch(100, 3, 4, g=6, fp8=True) == ("attn_group8_g6_t1_k16", (10, 4, 1), 192, 84480)
    assert refabi.flash_launch(100, 3, 4, g=6, mfma=True) == ("attn_mfma_g6_t2", (7, 4, 1), 768, 37376)
    assert refabi.flash_launch(100, 3, 8, g=1) == ("attn_group_g1_t8_k16", (4, 8, 1), 256, 101376)
    assert refabi.flash_launch(100, 3, 8, g=2, fp8=True) == ("attn_group8_g2_t4_k16", (5, 8, 1), 256, 101376)
    assert refabi.flash_launch(100, 3, 2, g=8) == ("attn_group_g8_t1_k16", (10, 2, 1), 256, 101376)


def test_reference_prompt_kernels_fit_lds(tmp_path):
    """Static LDS of each prompt kernel of the code object plus the dynamic
    shared memory the engine's launch passes (flash_launch, model.rs:58-79)
    fits one CU's 160 KiB; otherwise the dispatch is rejected."""
    import re
    import subprocess
    from pkv import refabi
    bundler = "/opt/rocm/llvm/bin/clang-offload-bundler"
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    co = tmp_path / "gfx950.co"
    subprocess.run([bundler, "--unbundle", "--type=o", f"--input={refabi.HSACO}", f"--output={co}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950"], check=True)
    notes = subprocess.run([readelf, "--notes", str(co)], check=True, capture_output=True, text=True).stdout
    static = {}
    for item in notes.split("\n  - ")[1:]:
        name = re.search(r"\.name:\s+(\S+)", item)
        lds = re.search(r"\.group_segment_fixed_size:\s+(\d+)", item)
        if name and lds:
            static[name.group(1)] = int(lds.group(1))
    for kw in ({}, {"mfma": True}, {"fp8": True}, {"g": 6}, {"g": 6, "fp8": True}, {"g": 1}, {"g": 2}, {"g": 8},
               {"g": 1, "fp8": True}, {"g": 2, "fp8": True}, {"g": 8, "fp8": True}):
        name, _, _, smem = refabi.flash_launch(100, 3, 4, **kw)
        assert name in static, (name, sorted(static))
        assert static[name] + smem <= 160 * 1024, (name, static[name], smem)
    # attn_groupr keeps its two K / V stages (K pairs 1,040 B, V pairs 1,056 B
    # apart, 16 pairs each) and 4 page-id rings of 64 B in the engine's
    # dynamic allocation, with no static LDS: two workgroups per CU
    name, _, _, smem = refabi.flash_launch(100, 3, 4)
    assert static[name] == 0 and 2 * smem <= 160 * 1024, (static[name], smem)
    assert smem >= 2 * (16 * 1040 + 16 * 1056) + 4 * 64, smem
