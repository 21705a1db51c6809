// Per-kernel resource figures of the fused kernels as the compiler reported
// them (-Rpass-analysis=kernel-resource-usage) when the library was built:
// the build turns the report into a table (a generated source file), so the
// resource query can give AGPRs and SGPRs, which hipFuncGetAttributes does
// not expose.
#pragma once

namespace fa {

struct KernelResources
{
    int head_dim;         // template parameter D
    int waves_per_group;  // kWpg
    int causal;           // kCausal
    int groups;           // kGroups
    int list;             // kList (two half blocks walked as one list)
    int vgprs;            // architectural VGPRs
    int agprs;            // accumulation VGPRs
    int sgprs;            // scalar registers (total)
    int lds_bytes;        // static LDS per workgroup
    int scratch_bytes;    // private (spill) bytes per lane
};

extern const KernelResources kFusedKernelResources[];
extern const int kFusedKernelResourceCount;

}  // namespace fa
