"""CPU tests of libfa_mi355x.so: it loads, exports every symbol the public
headers declare, and its host-side logic (FLOP / byte models, scale, argument
validation that returns before any HIP call) matches the oracle and the
reference's conventions. No kernel is launched here."""
import os
import re
import subprocess

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fa_mi355x.h")


def declared_c_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def exported_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_every_declared_symbol_is_exported(fa_lib):
    declared = declared_c_symbols()
    assert len(declared) == len(fa_lib._SIGNATURES), declared
    exported = exported_symbols(fa_lib.LIB_PATH)
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    L = fa_lib.lib()
    for s in declared:
        assert getattr(L, s) is not None


def test_cpp_interface_symbols_exported(fa_lib):
    """The C++ API of include/flash_attention.h is exported (mangled) too."""
    out = subprocess.run(["nm", "-DC", "--defined-only", fa_lib.LIB_PATH], check=True, capture_output=True,
                         text=True).stdout
    for name in ("launch_attention_unfused", "launch_softmax_rows_inplace", "launch_attention_tensorcore_v3",
                 "query_tensorcore_v3", "tensorcore_v3_hbm_bytes", "tensorcore_v3_supported", "attention_flops",
                 "unfused_workspace_bytes", "launch_attention_unfused_profile", "launch_attention_tensorcore_v3b",
                 "fused_row_supported", "query_fused_tiling", "launch_attention_fusedtiling_v2b"):
        assert f"cuda_op_lab::flash_attention::{name}(" in out, name


def walked_tiles_per_slab(bh, N, rows, groups, causal, cus=256):
    """K/V tiles the workgroups of one slab load, restated from
    fused_attention_kernel's walk (a workgroup's groups split one walk, so a
    tile counts once per workgroup that walks it): contiguous blocks walk the
    tiles up to their last key; a one-round causal grid pairs half blocks p
    and last - p, and a two-group workgroup walks up to its later half
    block's last key while the list layout (128 rows, four groups) walks the
    list "half block A's tiles, then half block B's"."""
    tile, half = 32, rows // 2
    lst = (rows, groups) == (128, 4)
    blocks = -(-N // rows)
    paired = causal and (groups == 2 or lst) and bh * blocks <= cus
    n_half = -(-N // half)
    q_blocks = (n_half + 1) // 2 if paired else blocks

    def half_tiles(r0):  # tiles the rows [r0, r0 + half) may see
        if r0 >= N:
            return 0
        return (min(r0 + half - 1, N - 1) if causal else N - 1) // tile + 1

    total = 0
    for qb in range(q_blocks):
        pa, pb = qb, n_half - 1 - qb
        if lst:
            a0 = pa * half if paired else qb * rows
            b0 = ((pb if pb > pa else n_half) * half) if paired else qb * rows + half
            total += half_tiles(a0) + half_tiles(b0)
        else:
            last_row = ((pb if pb > pa else pa) * half + half - 1) if paired else qb * rows + rows - 1
            last_key = min(last_row, N - 1) if causal else N - 1
            total += last_key // tile + 1
    return total


def test_host_models_match_oracle(fa_lib, oracle_mod):
    L = oracle_mod.lib()
    for (B, H, N, D) in [(1, 2, 128, 64), (2, 8, 2048, 64), (2, 8, 2048, 128), (4, 8, 8192, 128), (1, 16, 16384, 128),
                         (1, 1, 1, 64), (3, 5, 77, 128), (1, 8, 2048, 128), (1, 3, 1100, 64), (2, 4, 1000, 128),
                         (1, 1, 2049, 128), (1, 4, 8192, 64), (4, 8, 2048, 64), (8, 8, 1024, 64)]:
        shape = fa_lib.AttentionShape(B, H, N, D)
        for causal in (False, True):
            assert fa_lib.attention_flops(shape, causal) == oracle_mod.attention_flops(B, H, N, D, causal)
            # the model follows the configuration the v3 entry runs at this shape
            rows, groups = fa_lib.tensorcore_v3_config(shape, causal)
            assert (rows, groups) in ((64, 2), (64, 4), (128, 2), (128, 4), (256, 1))
            assert fa_lib.tensorcore_v3_rows_per_block(shape, causal) == rows
            for model, (r, g) in ((fa_lib.tensorcore_v3_hbm_bytes, (rows, groups)),
                                  (fa_lib.tensorcore_v3b_hbm_bytes, (64, 2))):
                tiles = walked_tiles_per_slab(B * H, N, r, g, causal)
                assert model(shape, causal) == 2 * B * H * N * D * 2 + 2 * B * H * tiles * 32 * D * 2, (shape, causal, r, g)
                contiguous = not causal or g not in (2, 4) or B * H * -(-N // r) > 256 or (g == 4 and r == 64)
                if contiguous:  # the reference's accounting, pinned to its published values
                    assert model(shape, causal) == L.fa_oracle_blocked_kv_hbm_bytes(B, H, N, D, int(causal), r, 32)
        assert fa_lib.unfused_workspace_bytes(shape) == L.fa_oracle_unfused_workspace_bytes(B, H, N)
    # one-round causal layouts load more than contiguous blocks would: c2
    # causal's list layout walks 1056 tiles per slab (16 pairs x 66) where 16
    # contiguous 128-row blocks would walk 544; c3's paired layout 784
    assert walked_tiles_per_slab(16, 2048, 128, 4, True) == 1056
    assert walked_tiles_per_slab(16, 2048, 128, 2, True) == 784
    assert walked_tiles_per_slab(16 * 64, 2048, 128, 2, True) == 544  # several rounds: contiguous
    c2c = fa_lib.AttentionShape(2, 8, 2048, 64)
    assert fa_lib.tensorcore_v3_hbm_bytes(c2c, True) == 2 * 16 * 2048 * 64 * 2 + 2 * 16 * 1056 * 32 * 64 * 2
    for d in (1, 3, 64, 80, 96, 128, 256):
        assert np.float32(fa_lib.default_scale(d)) == np.float32(oracle_mod.default_scale(d))


def test_error_state_records_host_side_rejections(fa_lib):
    """fa_get_last_error: a host-side rejection is kept for the calling thread
    until read (hipGetLastError semantics); an unsupported head_dim is silent;
    an empty shape is a success that leaves the state alone."""
    L = fa_lib.lib()
    fake = 0x10000
    assert fa_lib.get_last_error() in (0, 1)  # earlier tests may have left one
    assert fa_lib.get_last_error() == 0
    assert L.fa_launch_attention_tensorcore_v3(fake + 8, fake, fake, fake, 1, 1, 64, 64, 0, None) == 1
    assert fa_lib.peek_at_last_error() == 1 and fa_lib.peek_at_last_error() == 1
    assert L.fa_launch_attention_tensorcore_v3(None, None, None, None, 0, 8, 64, 64, 0, None) == 0
    assert fa_lib.get_last_error() == 1
    assert fa_lib.get_last_error() == 0
    assert L.fa_launch_attention_tensorcore_v3(fake, fake, fake, fake, 1, 1, 64, 96, 0, None) == fa_lib.FA_ERROR_UNSUPPORTED
    assert fa_lib.get_last_error() == 0
    assert L.fa_launch_attention_unfused(fake, fake, fake, fake, None, 1, 1, 64, 64, 0, None) == 1
    assert L.fa_launch_softmax_rows_inplace(None, 3, 10, None) == 1
    assert L.fa_query_fused(64, 96, None) == 1
    assert fa_lib.get_last_error() == 1 and fa_lib.get_last_error() == 0


def test_configuration_rule_without_a_device(fa_lib):
    """The v3 configuration rule on the CPU (the CU count falls back to an
    MI355X's 256): three of the four (2,8,2048,D) metric shapes run 128 rows
    in two groups and (2,8,2048,64) causal, one round of 128-row workgroups,
    the four-group list layout; small head_dim-64 grids take four KV groups;
    256 rows in one group where the rule's three cases apply; an unsupported
    head_dim reports no configuration."""
    for d in (64, 128):
        for causal in (False, True):
            want = (128, 4) if (d, causal) == (64, True) else (128, 2)
            assert fa_lib.tensorcore_v3_config((2, 8, 2048, d), causal) == want
    assert fa_lib.tensorcore_v3_config((4, 8, 1024, 64), True) == (128, 2)
    assert fa_lib.tensorcore_v3_config((1, 4, 8192, 64), True) == (128, 4)
    assert fa_lib.tensorcore_v3_config((1, 8, 2048, 64), True) == (64, 4)
    assert fa_lib.tensorcore_v3_config((1, 8, 512, 64), False) == (64, 2)
    assert fa_lib.tensorcore_v3_config((4, 8, 8192, 64), False) == (256, 1)
    assert fa_lib.tensorcore_v3_config((4, 8, 8192, 128), False) == (256, 1)
    assert fa_lib.tensorcore_v3_config((1, 8, 4096, 128), False) == (128, 2)   # 128 256-row workgroups
    assert fa_lib.tensorcore_v3_config((4, 8, 2048, 64), True) == (64, 2)
    # causal, 256 rows: long sequences with two rounds of them, or one round
    # of them replacing two rounds of 128-row workgroups at short lengths
    assert fa_lib.tensorcore_v3_config((2, 8, 8192, 64), True) == (256, 1)
    assert fa_lib.tensorcore_v3_config((1, 8, 8192, 128), True) == (128, 2)
    assert fa_lib.tensorcore_v3_config((16, 8, 512, 128), True) == (256, 1)
    assert fa_lib.tensorcore_v3_config((4, 8, 2048, 128), True) == (256, 1)
    assert fa_lib.tensorcore_v3_config((2, 8, 4096, 128), True) == (128, 2)
    assert fa_lib.tensorcore_v3_config((12, 8, 1024, 128), True) == (128, 2)  # 1.5 rounds of 256-row
    assert fa_lib.tensorcore_v3_config((8, 8, 1024, 64), True) == (256, 1)
    assert fa_lib.tensorcore_v3_config((4, 8, 2048, 64), True) == (64, 2)
    assert fa_lib.tensorcore_v3_config((1, 8, 512, 96), False) is None
    assert fa_lib.tensorcore_v3_rows_per_block((1, 8, 512, 96), False) == 0


def test_supported_head_dims(fa_lib):
    for d in (64, 128):
        assert fa_lib.tensorcore_v3_supported(d) and fa_lib.tensorcore_v3b_supported(d)
    for d in (0, 1, 32, 63, 65, 96, 127, 129, 256):
        assert not fa_lib.tensorcore_v3_supported(d) and not fa_lib.tensorcore_v3b_supported(d)


def test_argument_validation_before_launch(fa_lib):
    L = fa_lib.lib()
    fake = 0x10000  # never dereferenced: every call below returns before a launch
    # unsupported head_dim: nothing launched, FA_ERROR_UNSUPPORTED
    assert L.fa_launch_attention_tensorcore_v3(fake, fake, fake, fake, 1, 1, 64, 96, 0, None) == fa_lib.FA_ERROR_UNSUPPORTED
    assert L.fa_launch_attention_tensorcore_v3b(fake, fake, fake, fake, 1, 1, 64, 32, 1, None) == fa_lib.FA_ERROR_UNSUPPORTED
    # the four-group configurations exist at head_dim 64 only; unknown
    # (rows, groups) pairs are invalid
    for rows, groups in ((64, 4), (128, 4)):
        assert L.fa_launch_attention_fused_groups(fake, fake, fake, fake, 1, 1, 64, 128, 1, rows, groups,
                                                  None) == fa_lib.FA_ERROR_UNSUPPORTED
    for rows, groups in ((128, 1), (256, 2), (128, 3), (96, 4), (0, 2)):
        assert L.fa_launch_attention_fused_groups(fake, fake, fake, fake, 1, 1, 64, 64, 0, rows, groups, None) == 1
    # empty shapes are a successful no-op
    assert L.fa_launch_attention_tensorcore_v3(None, None, None, None, 0, 8, 64, 64, 0, None) == 0
    assert L.fa_launch_attention_tensorcore_v3(None, None, None, None, 1, 8, 0, 128, 1, None) == 0
    assert L.fa_launch_attention_unfused(None, None, None, None, None, 1, 0, 64, 64, 0, None) == 0
    assert L.fa_launch_softmax_rows_inplace(None, 0, 10, None) == 0
    # null pointers / negative dims / misaligned bases are rejected
    assert L.fa_launch_attention_tensorcore_v3(None, fake, fake, fake, 1, 1, 64, 64, 0, None) == 1
    assert L.fa_launch_attention_tensorcore_v3(fake, fake, fake, fake, -1, 1, 64, 64, 0, None) == 1
    assert L.fa_launch_attention_tensorcore_v3(fake + 2, fake, fake, fake, 1, 1, 64, 64, 0, None) == 1
    assert L.fa_launch_attention_unfused(fake, fake, fake, fake, None, 1, 1, 64, 64, 0, None) == 1
    assert L.fa_launch_attention_unfused(fake, fake, fake, fake, fake, 1, 1, 64, 0, 0, None) == 1
    assert L.fa_launch_softmax_rows_inplace(None, 3, 10, None) == 1
    assert L.fa_launch_softmax_rows_inplace(fake, -1, 10, None) == 1
    # one (batch, head) slab past 2^31 bytes: DMA offsets within a slab are 32-bit, so it is rejected
    assert L.fa_launch_attention_tensorcore_v3(fake, fake, fake, fake, 1, 1, 1 << 24, 128, 0, None) == 1
    assert L.fa_launch_attention_tensorcore_v3(fake, fake, fake, fake, 1, 1, 1 << 25, 64, 1, None) == 1
    # the pinned-configuration entry: only 0 (auto), 64, 128 and 256 rows per workgroup
    for rows in (-1, 1, 32, 96, 512):
        assert L.fa_launch_attention_fused(fake, fake, fake, fake, 1, 1, 64, 64, 0, rows, None) == 1
    assert L.fa_launch_attention_fused(None, None, None, None, 0, 8, 64, 64, 1, 256, None) == 0
    for rows in (0, 64, 128, 256):
        assert L.fa_launch_attention_fused(fake, fake, fake, fake, 1, 1, 64, 96, 0, rows, None) == fa_lib.FA_ERROR_UNSUPPORTED
        assert L.fa_launch_attention_fused(None, None, None, None, 0, 8, 64, 128, 1, rows, None) == 0
    # the Python mirror: unsupported -> False (silent, like the reference), errors raise
    shape = fa_lib.AttentionShape(1, 1, 64, 96)
    assert fa_lib.launch_attention_tensorcore_v3(fake, fake, fake, fake, shape, False, stream=0) is False
    with pytest.raises(fa_lib.FaError):
        fa_lib.launch_attention_tensorcore_v3(None, fake, fake, fake, (1, 1, 64, 64), False, stream=0)


def test_calibration_rejects_bad_arguments_before_any_device_call(fa_lib):
    """fa_mfma_peak checks its arguments on the host first (no launch)."""
    import ctypes

    L = fa_lib.lib()
    tf, ghz = ctypes.c_double(), ctypes.c_double()
    fake = 0x10000
    assert L.fa_mfma_peak(None, 4, 1, fake, ctypes.byref(tf), ctypes.byref(ghz), None) == 1  # < 8 MFMAs per wave
    assert L.fa_mfma_peak(None, 64, 0, fake, ctypes.byref(tf), ctypes.byref(ghz), None) == 1  # no launch
    assert L.fa_mfma_peak(None, 64, 1, None, ctypes.byref(tf), ctypes.byref(ghz), None) == 1  # no records
    assert fa_lib.get_last_error() == 1


def test_query_unsupported_needs_no_gpu(fa_lib):
    info = fa_lib.query_tensorcore_v3(96)
    assert info["supported"] == 0


def test_build_info(fa_lib):
    assert "gfx950" in fa_lib.build_info()


def test_cpp_header_compiles_as_drop_in(tmp_path, fa_lib):
    """A harness written against the reference interface compiles against
    include/flash_attention.h and links libfa_mi355x.so; it runs the host-only
    calls (no GPU needed)."""
    src = tmp_path / "dropin.cpp"
    src.write_text(r'''
#include "flash_attention.h"
#include "flash_attention_v0_profile.h"
#include <cstdio>
using namespace cuda_op_lab::flash_attention;
int main() {
    const AttentionShape shape{2, 8, 2048, 128};
    std::printf("%.0f %zu %d %d %.9g %d\n", attention_flops(shape, false), unfused_workspace_bytes(shape),
                (int)tensorcore_v3_supported(128), (int)fused_row_supported(64), default_scale(128),
                (int)query_fused_tiling(64).supported);
    void (*launch)(const __hip_bfloat16*, const __hip_bfloat16*, const __hip_bfloat16*, __hip_bfloat16*,
                   const AttentionShape&, bool, hipStream_t) = launch_attention_tensorcore_v3;
    return launch == nullptr;
}
''')
    exe = tmp_path / "dropin"
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    pkg = os.path.dirname(fa_lib.LIB_PATH)
    subprocess.run([hipcc, "-std=c++17", "-O1", f"-I{REPO}/include", str(src), "-o", str(exe), f"-L{pkg}",
                    "-lfa_mi355x", f"-Wl,-rpath,{pkg}"], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out[0] == "34359738368" and out[1] == str(2 * 8 * 2048 * 2048 * 4)
    assert out[2] == "1" and out[3] == "0" and out[5] == "0"
    assert np.float32(float(out[4])) == np.float32(1.0) / np.sqrt(np.float32(128))


def test_cpp_caller_sees_host_side_rejections(tmp_path, fa_lib):
    """A reference-style caller of the void C++ launchers sees a launch this
    library refuses on the host: a misaligned base and a slab past 2^31
    bytes (fused), a missing workspace (v0). The rejections happen before any
    HIP call, so no GPU is needed."""
    src = tmp_path / "dropin_errors.cpp"
    src.write_text(r'''
#include "flash_attention.h"
#include <cstdio>
#include <cstdint>
using namespace cuda_op_lab::flash_attention;
int main() {
    auto* base = reinterpret_cast<__hip_bfloat16*>(std::uintptr_t{0x10000});
    auto* misaligned = reinterpret_cast<__hip_bfloat16*>(std::uintptr_t{0x10008});
    int fails = 0;
    if (get_last_error() != hipSuccess) ++fails;                      // clean start
    launch_attention_tensorcore_v3(misaligned, base, base, base, AttentionShape{1, 1, 64, 64}, false);
    if (peek_at_last_error() != hipErrorInvalidValue) ++fails;        // visible, not consumed
    if (get_last_error() != hipErrorInvalidValue) ++fails;
    if (get_last_error() != hipSuccess) ++fails;                      // consumed
    launch_attention_tensorcore_v3(base, base, base, base, AttentionShape{1, 1, 1 << 24, 128}, true);
    if (get_last_error() != hipErrorInvalidValue) ++fails;            // one slab past 2^31 bytes
    launch_attention_tensorcore_v3b(base, base, base, misaligned, AttentionShape{2, 1, 64, 128}, false);
    if (get_last_error() != hipErrorInvalidValue) ++fails;
    launch_attention_unfused(base, base, base, base, nullptr, AttentionShape{1, 1, 64, 64}, false);
    if (get_last_error() != hipErrorInvalidValue) ++fails;            // v0 without a workspace
    launch_attention_tensorcore_v3(base, base, base, base, AttentionShape{1, 1, 64, 96}, false);
    if (get_last_error() != hipSuccess) ++fails;                      // unsupported head_dim: silent
    std::printf("%d\n", fails);
    return fails;
}
''')
    exe = tmp_path / "dropin_errors"
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    pkg = os.path.dirname(fa_lib.LIB_PATH)
    subprocess.run([hipcc, "-std=c++17", "-O1", f"-I{REPO}/include", str(src), "-o", str(exe), f"-L{pkg}",
                    "-lfa_mi355x", f"-Wl,-rpath,{pkg}"], check=True, capture_output=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0 and res.stdout.split() == ["0"], (res.stdout, res.stderr)


def test_traffic_record_hash_ignores_comments_only():
    """bench.py ties each HBM-traffic measurement (profiles/traffic.json) to
    a hash of the fused kernel's code: comments and blank lines do not
    change it; code and compiler flags do."""
    import bench

    code = "int a = 1;\nfloat f(float x) { return x * 2.0f; }\n"
    noted = "// note\nint a = 1;  /* old value 2\n */\n\nfloat f(float x) { return x * 2.0f; }  // doubled\n"
    assert bench.strip_cpp_comments(code) == bench.strip_cpp_comments(noted)
    assert bench.strip_cpp_comments(code) != bench.strip_cpp_comments(code.replace("2.0f", "3.0f"))
    sha = bench.kernel_source_sha()
    assert len(sha) == 16 and int(sha, 16) >= 0
