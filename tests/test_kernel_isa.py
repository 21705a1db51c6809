"""CPU checks on the gfx950 assembly of the fused kernels (hipcc cross-compiles
it here; no GPU needed).

The reference's resource contract says a kernel's local (spill) bytes "must be
0, or the output accumulator spilled" (include/flash_attention.h:51,68 of the
reference). One instantiation here, the dense head_dim-64 one-group kernel,
is compiled for two workgroups per CU (at most 128 VGPRs) and the compiler
spills a few values of it. This test pins where that traffic can be: no
scratch instruction of any fused kernel may lie inside a loop (the step walk,
the copy-only steps, the barrier padding), so a spill costs a few stores
before the walk and the same reloads after it, never per step. The compiler
marks every basic block inside a loop ("in Loop: Header=..." / "Loop
Header"), which is what the check reads.
"""
import os
import re
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "cuda_fused_attention_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"

_FUNC = re.compile(r"^(_Z\S*fused_attention_kernel\S*):")
_BLOCK = re.compile(r"^(\.LBB\d+_\d+:|; %bb\.\d+:)(.*)$")
# fused_attention_kernel<D, kWpg, kCausal, kGroups, kList>
_TEMPLATE = re.compile(r"fused_attention_kernelILi(\d+)ELi(\d+)ELb([01])ELi(\d+)ELb([01])EE")


def kernel_blocks(asm: str):
    """{kernel: [(in_loop, [instructions])]} for every fused kernel."""
    out, func, blocks = {}, None, None
    for line in asm.splitlines():
        m = _FUNC.match(line)
        if m:
            func = m.group(1)
            blocks = [(False, [])]
            out[func] = blocks
            continue
        if func is None:
            continue
        if line.startswith("\t.section") or line.startswith(".Lfunc_end"):
            func = None
            continue
        b = _BLOCK.match(line)
        if b:
            blocks.append(("in Loop" in b.group(2) or "Loop Header" in b.group(2), []))
            continue
        text = line.strip()
        if text and not text.startswith(";") and not text.startswith("."):
            blocks[-1][1].append(text.split()[0])
    return out


@pytest.fixture(scope="module")
def fused_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    sys.path.insert(0, REPO)
    from cuda_fused_attention_amd import _build

    out = tmp_path_factory.mktemp("isa") / "fa_fused.s"
    subprocess.run([HIPCC, *_build.HIP_FLAGS, f"-I{CSRC}", "--cuda-device-only", "-S", "-x", "hip",
                    os.path.join(CSRC, "fa_fused.hip"), "-o", str(out)], check=True, capture_output=True)
    return kernel_blocks(out.read_text())


def test_no_spill_traffic_in_step_loops(fused_asm):
    assert len(fused_asm) >= 16, sorted(fused_asm)
    spilling = []
    for func, blocks in fused_asm.items():
        t = _TEMPLATE.search(func)
        assert t, func
        d, wpg, causal, groups, lst = (int(x) for x in t.groups())
        loops = sum(1 for in_loop, _ in blocks if in_loop)
        assert loops > 0, ("no loop found: the block annotations changed", func)
        scratch_in_loop = [op for in_loop, ops in blocks if in_loop for op in ops if op.startswith("scratch_")]
        assert not scratch_in_loop, ((d, wpg, causal, groups, lst), scratch_in_loop)
        if any(op.startswith("scratch_") for _, ops in blocks for op in ops):
            spilling.append((d, wpg, causal, groups, lst))
    # only the dense head_dim-64 one-group build (capped at 128 VGPRs) may spill
    assert set(spilling) <= {(64, 8, 0, 1, 0)}, spilling


def test_loop_detection_sees_scratch_in_a_loop():
    """The parser flags a scratch access inside an annotated loop block
    (planted example in the compiler's annotation format)."""
    asm = ("_Z22fused_attention_kernelILi64ELi8ELb0ELi1ELb0EEvv:\n"
           "\tscratch_store_dword off, v1, off\n"
           ".LBB0_1:                                ; =>This Inner Loop Header: Depth=1\n"
           "\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]\n"
           "; %bb.2:                                ;   in Loop: Header=BB0_1 Depth=1\n"
           "\tscratch_load_dword v1, off, off\n"
           "\ts_cbranch_scc1 .LBB0_1\n"
           ".LBB0_3:\n"
           "\ts_endpgm\n")
    blocks = kernel_blocks(asm)["_Z22fused_attention_kernelILi64ELi8ELb0ELi1ELb0EEvv"]
    in_loop = [op for flag, ops in blocks if flag for op in ops]
    outside = [op for flag, ops in blocks if not flag for op in ops]
    assert "scratch_load_dword" in in_loop and "scratch_store_dword" in outside and "s_endpgm" in outside
