// k_gns.hip -- host side shared by the streaming GroupNorm launchers
// (k_gns_fwd.hip, k_gns_bwd.hip): shape plan, workspace clear
// and the persistent grid size.
#include <stdlib.h>

#include <atomic>

#include "gn_stream.h"

namespace nnk {
namespace gns {

static bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

Plan make_plan(bool bwd, int B, int HW, int C, int G) {
    Plan p{};
    p.ok = false;
    if (B <= 0 || HW <= 0 || C <= 0 || G <= 0 || C % G != 0) return p;
    const int cpg = C / G;
    if (cpg % 4 != 0) return p;
    const int cpg4 = cpg / 4;
    if (cpg4 != 1 && cpg4 != 2 && cpg4 != 4) return p;
    const int kCw4 = bwd ? kBwdCw4 : kFwdCw4;
    if (C % (4 * kCw4) != 0) return p;
    const int TP = bwd ? kBwdTp : kFwdTp;
    if (HW % TP != 0) return p;
    const int T = HW / TP;
    if (!is_pow2(T)) return p;
    const int GT = kCw4 / cpg4;
    // merging lanes per group: their xor tree runs inside one wave, and the
    // GT groups' mergers must fit in the workgroup
    const int lpg_max = kTpb / GT < kWave ? kTpb / GT : kWave;
    int rpl = 0;
    if (T <= lpg_max) rpl = 1;
    else if (T <= 2 * lpg_max) rpl = 2;
    else return p;
    if ((long long)HW * C * 4 >= (1LL << 31)) return p;
    const int NCB = C / (4 * kCw4);
    if ((long long)NCB * T > kMaxGrid) return p;
    if ((long long)B * NCB * T >= (1LL << 31) / (2 * GT)) return p;
    p.cpg4 = cpg4;
    p.rpl = rpl;
    p.sh.B = B;
    p.sh.HW = HW;
    p.sh.C = C;
    p.sh.G = G;
    p.sh.T = T;
    p.sh.NCB = NCB;
    p.sh.ntiles = B * NCB * T;
    p.sh.sample_bytes = (uint32_t)((long long)HW * C * 4);
    p.sh.inv_n = 1.0f / (float)((long long)HW * cpg);
    static_assert(kCountOffset + (kMaxGrid + 1) * sizeof(unsigned) <= kHeaderBytes, "counters fit the header");
    p.rec_offset = kHeaderBytes;
    const size_t rec_bytes = (size_t)p.sh.ntiles * GT * 2 * sizeof(unsigned long long);
    // backward partials: one [2][4 * kCw4] block per workgroup and per team
    const size_t nval_bytes = (size_t)2 * (4 * kCw4) * sizeof(unsigned long long);
    p.part_offset = p.rec_offset + rec_bytes;
    const size_t part_bytes = bwd ? (size_t)kMaxGrid * nval_bytes : 0;
    p.tpart_offset = p.part_offset + part_bytes;
    const size_t tpart_bytes = bwd ? (size_t)((kMaxGrid + T - 1) / T) * nval_bytes : 0;
    p.ws_floats = (p.tpart_offset + tpart_bytes + sizeof(float) - 1) / sizeof(float);
    // after everything epoch-tagged, on a 256-byte boundary: [tile][4 * kCw4]
    p.colpart_offset = (p.ws_floats * sizeof(float) + 255) / 256 * 256;
    p.ws_shift_floats =
        bwd ? p.colpart_offset / sizeof(float) + (size_t)p.sh.ntiles * 4 * kCw4 : p.ws_floats;
    p.ok = true;
    return p;
}

}  // namespace gns
}  // namespace nnk

namespace {

// Zero a workspace drawn from the stream-ordered pool before its first use.
__global__ void gns_clear(unsigned* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

}  // namespace

void nnk_clear_workspace(float* ws, size_t n_floats, hipStream_t s) {
    if (n_floats == 0) return;
    const size_t blocks = (n_floats + 255) / 256 < 4096 ? (n_floats + 255) / 256 : 4096;
    gns_clear<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(reinterpret_cast<unsigned*>(ws), n_floats);
}

// Polls of one statistics record before a wait gives up: kSpinLimit, or
// NNHIP_GN_SPIN_LIMIT when it is a number no larger (read per launch, so a
// test can force the wait-failure path: 0 makes every launch flag itself).
unsigned nnk_gns_spin_limit() {
    const char* e = getenv("NNHIP_GN_SPIN_LIMIT");
    if (!e || !*e) return nnk::gns::kSpinLimit;
    char* end = nullptr;
    const unsigned long v = strtoul(e, &end, 10);
    return (end && *end == '\0' && v <= nnk::gns::kSpinLimit) ? (unsigned)v : nnk::gns::kSpinLimit;
}

// Launch a persistent grid: a plain launch (its progress does not depend on
// residency; see gn_stream.h), or a cooperative one with
// NNHIP_GN_COOPERATIVE=1 for callers that run streaming GroupNorms
// concurrently on several streams.
bool nnk_gns_launch(const void* fn, int P, void** args, hipStream_t s, const char* what) {
    const char* e = getenv("NNHIP_GN_COOPERATIVE");
    const bool coop = e && e[0] == '1';
    const hipError_t r = coop ? hipLaunchCooperativeKernel(fn, dim3((unsigned)P), dim3(nnk::gns::kTpb), args, 0, s)
                              : hipLaunchKernel(fn, dim3((unsigned)P), dim3(nnk::gns::kTpb), args, 0, s);
    if (r != hipSuccess) {
        (void)hipGetLastError();
        nnk_path_note("%s: %s launch of %d x %d: %s", what, coop ? "cooperative" : "plain", P, nnk::gns::kTpb,
            hipGetErrorString(r));
        return false;
    }
    return true;
}

// Persistent grid size for a kernel: resident workgroups of the device
// (cached per device and kernel), capped and rounded down to whole units.
int nnk_gns_grid(const void* fn, int key, size_t lds, int unit) {
    constexpr int kDev = 16, kKeys = 2 * nnk::gns::kGnsBwdKeys;
    // per device and kernel: 0 = not yet queried, -1 = unusable, else the
    // resident workgroups per CU (relaxed atomics: concurrent callers may both
    // query, and store the same value)
    static std::atomic<int> occ_cache[kDev][kKeys];
    static std::atomic<int> cu_cache[kDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDev || key < 0 || key >= kKeys) return 0;
    if (occ_cache[dev][key].load(std::memory_order_relaxed) == 0) {
        const hipError_t ea =
            lds ? hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) : hipSuccess;
        if (ea != hipSuccess) {
            (void)hipGetLastError();
            nnk_path_note("streaming GroupNorm kernel %d: LDS attribute of %zu bytes: %s", key, lds,
                hipGetErrorString(ea));
            occ_cache[dev][key].store(-1, std::memory_order_relaxed);
            return 0;
        }
        int occ = 0;
        const hipError_t eo = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, nnk::gns::kTpb, lds);
        if (eo != hipSuccess || occ <= 0) {
            (void)hipGetLastError();
            nnk_path_note("streaming GroupNorm kernel %d: occupancy %d (%s)", key, occ, hipGetErrorString(eo));
            occ_cache[dev][key].store(-1, std::memory_order_relaxed);
            return 0;
        }
        occ_cache[dev][key].store(occ, std::memory_order_relaxed);
    }
    const int occ = occ_cache[dev][key].load(std::memory_order_relaxed);
    if (occ < 0) return 0;
    if (cu_cache[dev].load(std::memory_order_relaxed) == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
            (void)hipGetLastError();
            return 0;
        }
        cu_cache[dev].store(cus, std::memory_order_relaxed);
    }
    const int cus = cu_cache[dev].load(std::memory_order_relaxed);
    long long P = (long long)occ * cus;
    if (P > nnk::gns::kMaxGrid) P = nnk::gns::kMaxGrid;
    P = P / unit * unit;
    if (P <= 0)
        nnk_path_note("streaming GroupNorm kernel %d: %d resident workgroups < %d tiles per sample row", key,
            occ * cus, unit);
    return (int)P;
}
