// gn_stream.h -- streaming NHWC GroupNorm (+ fused activation) for large
// tensors: the HBM-bound path of the GroupNorm launchers.
//
// Reference maths: src/kernels.cu:622-717 (forward statistics, backward-x,
// backward-param), composed with the activation of src/kernels.cu:21-68 as the
// DDPM block does (src/conv_residual.c:28-29, 51-52).
//
// Why a streaming design.  A workgroup that holds a whole (sample, group) reads
// it as cpg-float columns of every pixel row (32 bytes per 1 KB row at the
// north-star shape) and runs load -> reduce -> store in lock-step phases; both
// cost bandwidth on gfx950.  Here every wave instruction reads whole 128-byte
// lines of contiguous pixel-row segments, and the group statistics of a sample
// are combined across workgroups without anyone blocking on them:
//
//   tile       = TP pixel rows x CW4 float4 columns (a column block) of one
//                sample; it covers GT = CW4 / (cpg/4) whole groups.  In the
//                forward the rows of pixel tile t are t, t + T, t + 2T, ...
//                (T tiles per sample), so the tiles streamed together read
//                neighbouring rows; the backward's tiles are row blocks.
//   grid       = P persistent workgroups (as many as the device holds at
//                once), P a multiple of the tiles per sample, so workgroup w
//                always owns the same (column block, pixel tile) position and
//                walks the samples; tile i = round * P + w.  The T workgroups
//                that own the tiles of one (sample, column block) are
//                consecutive: a team.
//   round j    : take tile j (this workgroup's tile w + j * P) from its LDS
//                stage buffer into registers and start the direct-to-LDS
//                loads of tile j+2 into that buffer (two stage buffers, so
//                two tiles are in flight while a round computes);
//                phase A on tile j (registers): per-group partial statistics
//                -> one epoch-tagged 64-bit record per (tile, group, value);
//                phase B on tile j-2 (kept in registers since round j-2):
//                read the T records of each of its groups, merge them in a
//                fixed order, normalise / form dx, store.
//
// The tiles awaiting phase B stay in VGPRs, the stage is read with explicit
// waits on the in-order vector-memory counter (the compiler does not track
// direct-to-LDS loads into two buffers), and the workgroup barriers wait for
// LDS operations only, so the staged loads stay in flight through phases A
// and B.  Each lane reads back exactly the stage slot its own load wrote, so
// the stage needs no barrier.  Phase B lags phase A by two rounds: a tile's
// records have two rounds to arrive, so the exchange round trip stays off the
// critical path.
//
// Records carry the launch epoch in their upper 32 bits and are written and
// read with agent-scope atomic 64-bit accesses, so a reader accepts exactly
// this launch's values and needs no fence or counter.  Every wait is bounded:
// past `spin_limit` polls the workgroup flags an error in the workspace and
// stops waiting (the kernel always terminates).
//
// Progress without a residency guarantee (plain launch).  A workgroup waits
// only for records of its own team, of the current or an earlier round, and
// never for anything else.  Workgroups are dispatched in index order on each
// XCD, so the resident workgroups of each XCD are a prefix of its share of
// the grid minus those already finished; the lowest unfinished team's members
// are therefore resident or next in line on every XCD, and what holds the
// slots they wait for either belongs to that team or is other work that ends
// by itself.  That team completes, and by induction so does the grid.  On an
// idle device all P workgroups are resident from the start.  Two streaming
// launches running concurrently on different streams could each hold slots the
// other's lowest team needs; the bounded wait then flags the error instead of
// hanging, and NNHIP_GN_COOPERATIVE=1 selects cooperative launches (all P
// resident by contract, at ~20 us more per launch) for such callers.
//
// Forward statistics are Chan et al.'s parallel mean/M2 merges of two-pass
// per-thread values (more accurate than the reference's E[x^2]-mu^2).  The
// backward sums S1 = sum g, S2 = sum g*xhat (g = dy*act'(h)*gamma) per group and
// accumulates the dgamma/dbeta partials per lane across the workgroup's tiles.
// dgamma/dbeta then need no wait either: the last workgroup of a team to
// arrive (an arrival counter) adds the team's partials in member order, and
// the last team to finish adds the team totals in team order; arrival order
// decides who adds, never the order of the additions.
#pragma once

#include <type_traits>

#include "nnk_common.h"

namespace nnk {
namespace gns {

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sample_rsrc(const float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)bytes, 0x00020000);
}

// Direct-to-LDS 128-bit buffer load: lane i of the wave reads 16 bytes at
// voff + soff and writes them to wave_slots + i (wave_slots uniform over the
// wave).  NT sets cache policy nt (bit 1) for inputs streamed once.
constexpr int kCpolNt = 2;
template <bool NT>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, float4* wave_slots, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)wave_slots, 16, (int)voff, (int)soff, 0, NT ? kCpolNt : 0);
}

// Workgroup barrier for LDS traffic: waits for this wave's LDS operations but
// not for its vector-memory loads, so the direct-to-LDS loads of the next tile
// stay in flight across it (__syncthreads' release fence would wait for them:
// they write LDS).  The signal fences keep the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maximum
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most N vector-memory operations of this wave are
// outstanding.  They complete in issue order, so this waits for everything
// issued before the last N.  The tile loops read the stage with inline
// assembly that the compiler does not track, so each round waits for its
// stage buffer explicitly, with N = the vector-memory operations that every
// wave issues after that buffer's loads (see the tile loops); a wave that
// issued more (conditional record stores, record polls) waits for more, never
// for less.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef __attribute__((address_space(3))) float4 lds_float4;
__device__ __forceinline__ uint32_t lds_addr(const float4* p) {
    return (uint32_t)(uintptr_t)(const lds_float4*)p;
}

// This lane's four 16-byte stage slots at addr + k * 16 KiB (k = 0..3; the
// slot stride of a 1024-thread workgroup), read and waited for in one
// statement so that no use of v is scheduled before the data is there.
__device__ __forceinline__ void lds_take4(float4 (&v)[4], uint32_t addr) {
    f32x4 a, b, c, d;
    asm volatile(
        "ds_read_b128 %0, %4\n\t"
        "ds_read_b128 %1, %4 offset:16384\n\t"
        "ds_read_b128 %2, %4 offset:32768\n\t"
        "ds_read_b128 %3, %4 offset:49152\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d)
        : "v"(addr)
        : "memory");
    v[0] = make_float4(a.x, a.y, a.z, a.w);
    v[1] = make_float4(b.x, b.y, b.z, b.w);
    v[2] = make_float4(c.x, c.y, c.z, c.w);
    v[3] = make_float4(d.x, d.y, d.z, d.w);
}

// lds_take4 plus the 16-byte shift slot at zaddr, added to v[0..NX) (the x
// part of the tile) once all five reads have landed.
template <int NX>
__device__ __forceinline__ void lds_take4_shift(float4 (&v)[4], uint32_t addr, uint32_t zaddr) {
    f32x4 a, b, c, d, z;
    asm volatile(
        "ds_read_b128 %0, %5\n\t"
        "ds_read_b128 %1, %5 offset:16384\n\t"
        "ds_read_b128 %2, %5 offset:32768\n\t"
        "ds_read_b128 %3, %5 offset:49152\n\t"
        "ds_read_b128 %4, %6\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d), "=&v"(z)
        : "v"(addr), "v"(zaddr)
        : "memory");
    v[0] = make_float4(a.x, a.y, a.z, a.w);
    v[1] = make_float4(b.x, b.y, b.z, b.w);
    v[2] = make_float4(c.x, c.y, c.z, c.w);
    v[3] = make_float4(d.x, d.y, d.z, d.w);
#pragma unroll
    for (int k = 0; k < NX; ++k) {
        v[k].x += z.x;
        v[k].y += z.y;
        v[k].z += z.z;
        v[k].w += z.w;
    }
}

// Make v's loads complete here.  Values loaded before the tile pipeline and
// used inside it would otherwise make the compiler's wait at their first use
// inside the loop a full vector-memory wait, i.e. a wait for the staged tile.
__device__ __forceinline__ void settle(const float4& v) {
    asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
}

// Same for prefetched records, on every lane of the wave: a prefetch that
// stays pending on lanes that never consume it makes the compiler fully drain
// the vector-memory counter before it reuses those registers.
template <int N>
__device__ __forceinline__ void settle(const unsigned long long (&r)[N]) {
#pragma unroll
    for (int u = 0; u < N; ++u) asm volatile("" ::"v"(r[u]));
}

// Chan merge of (na, ma, qa) with (nb, mb, qb).
__device__ __forceinline__ void chan_merge(float& n, float& m, float& q, float nb, float mb, float qb) {
    const float nn = n + nb;
    const float d = mb - m;
    m = m + d * (nb / nn);
    q = q + qb + d * d * (n * nb / nn);
    n = nn;
}
// Merge of two equal-count partials (count c each).
__device__ __forceinline__ void chan_merge_eq(float& m, float& q, float mo, float qo, float c) {
    const float d = mo - m;
    m = 0.5f * (m + mo);
    q = q + qo + d * d * (0.5f * c);
}

// ---------------------------------------------------------------------------
// Geometry shared by the forward and backward kernels.
// ---------------------------------------------------------------------------
template <int TPB_, int TP_, int CW4_, int CPG4_>
struct Geom {
    static constexpr int TPB = TPB_;            // threads per workgroup
    static constexpr int NW = TPB / kWave;      // waves
    static constexpr int TP = TP_;              // pixel rows per tile
    static constexpr int CW4 = CW4_;            // float4 columns per tile row
    static constexpr int CPG4 = CPG4_;          // float4 per group
    static constexpr int RW = kWave / CW4;      // tile rows per wave instruction
    static constexpr int RSTEP = NW * RW;       // tile rows per workgroup instruction
    static constexpr int NV = TP / RSTEP;       // float4 per thread per tensor
    static constexpr int GT = CW4 / CPG4;       // groups per tile
    static_assert(kWave % CW4 == 0 && CW4 % CPG4 == 0, "tile columns");
    static_assert(TP % RSTEP == 0 && NV >= 1, "tile rows");
    static_assert(GT <= kWave, "groups per tile");
};

// Runtime shape of a launch.
struct Shape {
    int B, HW, C, G;   // batch, pixels, channels, groups
    int T;             // pixel tiles per sample = HW / TP
    int NCB;           // column blocks per row = C / (4 * CW4)
    int ntiles;        // B * NCB * T
    uint32_t sample_bytes;
    float inv_n;       // 1 / (HW * cpg)
};

// Workspace layout (device), byte offsets:
//   0      err u32 (sticky wait-timeout flag)
//   4      epoch u32: the tag of the last launch on this workspace, advanced by
//          that launch's last workgroup (see launch_epoch)
//   256    arrival counters u32: [0] teams (backward) or workgroups (forward)
//          done, [1 + team] members done; zero between launches (each launch
//          re-arms what it counted)
//   8192   records u64, then (backward) the dgamma/dbeta partials.
// The header has a fixed size, so a workspace lent for one shape and then
// another never finds a counter where records were.
constexpr size_t kHeaderBytes = 8192;
constexpr size_t kCountOffset = 256;
struct Work {
    unsigned* err;             // the workspace's sticky timeout word
    unsigned* hflag;           // the process-wide host-mapped timeout word (or err)
    unsigned* ep;              // the epoch of the last launch on this workspace (0: none yet)
    unsigned* count;
    unsigned long long* rec;   // ntiles * GT * 2, [sample, column block][group][value][pixel tile]
    unsigned long long* part;  // bwd: [P][2][4 * CW4] per-workgroup dgamma/dbeta partials (tagged)
    unsigned long long* tpart; // bwd: [P / T][2][4 * CW4] per-team sums (tagged)
};

// The tag of this launch: one more than the last launch's on this workspace
// (never 0, the value of a zero-filled workspace).  Every workgroup reads the
// word at its start; only the launch's last workgroup, once every workgroup
// has arrived at the end (and so has read it), stores the new value.  The
// tag is therefore unique per launch on the workspace also when the launch
// is replayed from a captured graph with the same arguments.
__device__ __forceinline__ unsigned epoch_word(const Work& wk) {
    return __hip_atomic_load(wk.ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned epoch_of(unsigned word) {
    const unsigned e = word + 1u;
    return e ? e : 1u;
}
__device__ __forceinline__ unsigned launch_epoch(const Work& wk) { return epoch_of(epoch_word(wk)); }
__device__ __forceinline__ void publish_epoch(const Work& wk, unsigned epoch) {
    __hip_atomic_store(wk.ep, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One level of an xor reduction tree without LDS traffic: this lane's value
// and its partner's at lane distance O, as (lo, hi).  Every merge below is
// symmetric in its two operands (a + b, and Chan's equal-count merge), so
// both lanes of a pair compute the same bits, exactly as with __shfl_xor.
//   O = 1, 2: DPP quad permutes (the xor partner itself);
//   O = 4, 8: DPP mirrors within 8 and 16 lanes; the mirrored lane holds the
//     xor partner's value because the tree has already made every aligned
//     group of O lanes uniform (the levels below O run first);
//   O = 16, 32: the row swaps v_permlane16/32_swap (lo = the lower lane's value).
template <int O>
__device__ __forceinline__ void xpair(float v, float& lo, float& hi) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8 || O == 16 || O == 32, "xor distance");
    if constexpr (O <= 8) {
        constexpr int ctl = O == 1 ? 0xB1 : O == 2 ? 0x4E : O == 4 ? 0x141 : 0x140;
        lo = v;
        hi = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctl, 0xF, 0xF, false));
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    }
}
template <int O>
using xlevel = std::integral_constant<int, O>;

// The levels 1, 2, 4, ... n/2 of a tree over aligned groups of n lanes (n a
// power of two <= 64, uniform over the wave), smallest first: f(xlevel<O>).
template <class F>
__device__ __forceinline__ void for_xor_levels(int n, F f) {
    if (n > 1) f(xlevel<1>{});
    if (n > 2) f(xlevel<2>{});
    if (n > 4) f(xlevel<4>{});
    if (n > 8) f(xlevel<8>{});
    if (n > 16) f(xlevel<16>{});
    if (n > 32) f(xlevel<32>{});
}

// A run-time tree size as a scalar the compiler cannot see through, taken
// inside the tile loop: the level tests above then stay scalar compares and
// branches on it.  In the forward's loop the tests were otherwise hoisted
// out as lane masks, which ran out of scalar registers and came back
// through vector-lane spills (four vector instructions per level and round).
__device__ __forceinline__ int lpg_scalar(int n) {
    asm volatile("" : "+s"(n));
    return n;
}

// Lanes that share this lane's group inside a wave: the column bits inside
// the group (levels 1 .. CPG4 / 2), then the row bits of the wave (CW4 .. 32).
template <class Gm, class F>
__device__ __forceinline__ void for_group_xor(F f) {
    static_assert(Gm::CW4 == 16 || Gm::CW4 == 32, "row levels of the group tree");
    if constexpr (Gm::CPG4 > 1) f(xlevel<1>{});
    if constexpr (Gm::CPG4 > 2) f(xlevel<2>{});
    if constexpr (Gm::CW4 <= 16) f(xlevel<16>{});
    f(xlevel<32>{});
}

// a + (the partner's a) for each of the values, at one tree level
template <int O>
__device__ __forceinline__ void xsum(float& a) {
    float lo, hi;
    xpair<O>(a, lo, hi);
    a = lo + hi;
}
template <int O>
__device__ __forceinline__ void xmerge_eq(float& m, float& q, float c) {
    float ml, mh, ql, qh;
    xpair<O>(m, ml, mh);
    xpair<O>(q, ql, qh);
    m = ml;
    q = ql;
    chan_merge_eq(m, q, mh, qh, c);
}

// Slot of wave w's partial pair of group g in the per-tile exchange
// float2 [GT][NW].  The LDS has 64 four-byte banks, so a group's NW = 16
// pairs cover 32 banks and groups g, g + 1 together cover all 64.  The
// group leaders of one wave store at once (one lane per group); xoring the
// slot with g / 2 sends them to distinct banks (at the plain index w every
// even group would hit the same two banks).  The NW lanes that read one
// group back still read a permutation of its 16 pairs.
template <class Gm>
__device__ __forceinline__ int wave_slot(int g, int w) {
    static_assert((Gm::NW & (Gm::NW - 1)) == 0, "the slot xor needs a power-of-two wave count");
    return w ^ ((g >> 1) & (Gm::NW - 1));
}

// ---------------------------------------------------------------------------
// Forward.
// ---------------------------------------------------------------------------
// SHIFT: normalise x + shift[b, c] (a per-sample, per-channel term broadcast
// over the pixels, added to each tile as it is taken; x is not modified).
template <class Gm, int ACT, int RPL, bool NT, bool SHIFT>
__global__ __launch_bounds__(Gm::TPB) void gns_fwd(float* __restrict__ y, float* __restrict__ mu_out,
    float* __restrict__ rstd_out, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ shift, Shape sh, Work wk, float eps,
    unsigned spin_limit) {
#pragma clang fp contract(fast)
    constexpr int NW = Gm::NW, NV = Gm::NV, GT = Gm::GT, TPB = Gm::TPB, CW4 = Gm::CW4;
    static_assert(NV == 4 && TPB * 16 == 16384, "stage slots as lds_take4 reads them");
    // Tile rows interleaved one by one (RC = 1): same-box A/B at the
    // north-star shape 365 -> 347 us against contiguous tiles.
    constexpr int RC = 1;
    // Two stage buffers: the tiles of the next two rounds, written by
    // direct-to-LDS loads (round j takes buffer j % 2).  The tiles awaiting
    // phase B stay in registers.
    __shared__ float4 stage[2][NV * TPB];
    static_assert(2 * CW4 == kWave, "a wave's shift load covers the column block twice");
    __shared__ float4 shs[SHIFT ? 4 : 1][SHIFT ? kWave : 1];  // with SHIFT: the shift ring
    // Double-buffered by loop parity pb: consecutive phase A's (and phase B's)
    // may run with no barrier between them (first and last rounds), so a
    // buffer is rewritten only two phases later, past the other phase's barrier.
    __shared__ float2 wred[2][GT][NW];          // [parity][group][wave slot] (mean, M2)
    __shared__ float2 stat[2][GT];              // (mean, rstd)
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    // the wave index as a scalar: the direct-to-LDS loads take their LDS
    // address from a scalar register (M0), computed once per address
    const int wid_s = __builtin_amdgcn_readfirstlane(wid);
    const int col = lane % CW4, row0 = wid * Gm::RW + lane / CW4;
    const int gl = col / Gm::CPG4;              // group of this lane within the tile
    const int P = gridDim.x, w = blockIdx.x;
    const int T = sh.T, NCB = sh.NCB;
    const int cb = (w / T) % NCB;               // fixed column block of this workgroup
    const int t = w % T;                        // fixed pixel tile of this workgroup
    const int c0 = cb * CW4 * 4 + col * 4;      // first channel of this lane
    // The rows of a tile: RC consecutive rows at a time, tile t taking chunk t
    // of every T chunks.  The T tiles of a sample and column block partition
    // its rows for any RC, and the statistics merge over all of them; with
    // RC = 1 the tiles a team streams at once read neighbouring rows rather
    // than T separate blocks.
    static_assert(RC == Gm::TP || Gm::RSTEP % RC == 0, "row chunks");
    // local row r of tile t -> sample row (r / RC) T RC + t RC + r % RC
    const int lrow = (row0 / RC) * T * RC + row0 % RC;  // this lane's first row, tile 0
    constexpr bool kContig = RC == Gm::TP;
    const uint32_t voff = (uint32_t)(lrow * sh.C + c0) * 4u;
    const uint32_t rstep_rows = (uint32_t)(kContig ? Gm::RSTEP : Gm::RSTEP * T);
    const uint32_t rstep_bytes = rstep_rows * (uint32_t)sh.C * 4u;
    const uint32_t row_bytes = (uint32_t)sh.C * 4u;
    // gamma and beta of this lane's channels, loaded once the first tile's
    // loads are out (at the tile loop's start)
    float4 gm = make_float4(0.0f, 0.0f, 0.0f, 0.0f), bt = gm;
    const float nthr = (float)(NV * 4);
    const unsigned epoch = launch_epoch(wk);
    const unsigned long long tag = (unsigned long long)epoch << 32;
    const WaitFail wf{wk.err, wk.hflag};
    // A spin limit of 0 lets no wait succeed: the launch flags itself as
    // timed out (the error path, forced from the host for its tests).
    if (spin_limit == 0 && blockIdx.x == 0 && threadIdx.x == 0) wait_failed(wf);
    // merge role in phase B: LPG = T / RPL lanes per group (a power of two, at
    // most one wave and TPB / GT, so a group's mergers share a wave); lane rj
    // merges records rj, rj + LPG, ... (RPL of them)
    const int LPG = T / RPL;
    const int rg = tid / LPG, rj = tid % LPG;
    const bool merger = rg < GT;
    const int nt = sh.ntiles;

    // Round j works on this workgroup's tile w + j * P.  P is a multiple of
    // NCB * T (the tiles of one sample), so the tile's sample and its unit
    // (sample * NCB + column block) advance by constants from round to round.
    const int b0 = w / (NCB * T), spr = P / (NCB * T);
    const int u0 = w / T, upr = P / T;
    auto real_of = [&](int j) { return w + j * P < nt; };
    // Record layout [unit][group][value][pixel tile]: the mergers of a group
    // read consecutive tiles, i.e. contiguous records.
    auto rec_slot = [&](int j, int g, int tt) { return wk.rec + ((size_t)((u0 + j * upr) * GT + g) * 2) * T + tt; };
    // The same addresses as per-lane bases plus a uniform step per round, so
    // the tile loop adds one scalar offset instead of redoing the index
    // arithmetic: the merging lane's first record (group rg, or GT - 1 past
    // the mergers; tile rj) and the group leader's own (group tid / NW; tile t).
    const size_t rec_round = (size_t)upr * GT * 2 * T;
    const unsigned long long* const rec_m = rec_slot(0, merger ? rg : GT - 1, rj);
    unsigned long long* const rec_s = rec_slot(0, tid / NW < GT ? tid / NW : GT - 1, t);
    // With SHIFT the input is x + shift[b, c]: the 128 shift values of a
    // tile's sample and column block go into slot j % 4 of a small LDS ring
    // with one direct-to-LDS load per wave, issued just before the tile's own
    // loads (so the stage wait covers it), and are added to the tile as it is
    // taken.  Every wave writes the same values to the same slot: a wave reads
    // the slot only after its own load has landed, and a slot is rewritten
    // (tile j + 4) only after every wave has passed the barriers of the
    // rounds that read it (tile j).  A tile past the end reloads the last sample's shift.
    // One resource over the whole [B, C] shift for the kernel; the sample
    // moves the scalar offset (a tile past the end reads the last sample's).
    const __amdgpu_buffer_rsrc_t shr = sample_rsrc(shift, SHIFT ? (uint32_t)(sh.B * sh.C * 4) : 0u);
    const uint32_t shv = (uint32_t)(cb * CW4 * 4 + col * 4) * 4u;
    auto issue_shift = [&](int j) {
        if constexpr (SHIFT)
            dma16<false>(shr, &shs[j & 3][0], shv, (uint32_t)(real_of(j) ? b0 + j * spr : sh.B - 1) * row_bytes);
    };
    // The NV loads of round j's tile into stage buffer sb.  A tile past the
    // end is issued against an empty buffer range: the loads read nothing and
    // only keep the operation count of every round the same.
    auto issue = [&](int j, int sb) {
        const bool real = real_of(j);
        const __amdgpu_buffer_rsrc_t r =
            sample_rsrc(x + (size_t)(real ? b0 + j * spr : 0) * sh.HW * sh.C, real ? sh.sample_bytes : 0u);
        const uint32_t base = (uint32_t)(t * RC) * row_bytes;
        issue_shift(j);
#pragma unroll
        for (int k = 0; k < NV; ++k)
            dma16<NT>(r, &stage[sb][k * TPB + wid_s * kWave], voff, base + (uint32_t)k * rstep_bytes);
    };
    auto take = [&](float4 (&v)[NV], int j) {
        if constexpr (SHIFT)
            lds_take4_shift<NV>(v, lds_addr(&stage[j & 1][tid]), lds_addr(&shs[j & 3][col]));
        else
            lds_take4(v, lds_addr(&stage[j & 1][tid]));
    };
    auto phase_a = [&](float4 (&v)[NV], int j, int pb) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
        float m = s / nthr, q = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            q = fmaf(v[k].x - m, v[k].x - m, q);
            q = fmaf(v[k].y - m, v[k].y - m, q);
            q = fmaf(v[k].z - m, v[k].z - m, q);
            q = fmaf(v[k].w - m, v[k].w - m, q);
        }
        float cnt = nthr;
        for_group_xor<Gm>([&](auto o) {
            xmerge_eq<decltype(o)::value>(m, q, cnt);
            cnt *= 2.0f;
        });
        if (lane % CW4 % Gm::CPG4 == 0 && lane < CW4) wred[pb][gl][wave_slot<Gm>(gl, wid)] = make_float2(m, q);
        lds_barrier();
        // the NW wave partials of group g merge on lanes (g, i = 0..NW-1) of
        // one wave in a fixed xor tree (the merge is symmetric, so every lane
        // of the pair holds the same value)
        static_assert(kWave % NW == 0 && GT * NW % kWave == 0, "a group's wave partials share a wave");
        if (tid < GT * NW) {  // whole waves: GT * NW is a multiple of 64
            const int g = tid / NW, i = tid % NW;
            const float2 pq = wred[pb][g][wave_slot<Gm>(g, i)];
            float mm = pq.x, qq = pq.y;
            for_xor_levels(NW, [&](auto o) {
                xmerge_eq<decltype(o)::value>(mm, qq, cnt);
                cnt *= 2.0f;
            });
            if (i == 0) {
                unsigned long long* r = rec_s + (size_t)j * rec_round;
                rec_store(r, tagged(tag, mm));
                rec_store(r + T, tagged(tag, qq));
            }
        }
    };
    // Every lane loads (lanes past the mergers read group GT-1 and ignore it):
    // a branch here would put a path without these loads in front of the
    // record waits.
    unsigned long long r0[RPL] = {}, r1[RPL] = {};
    auto records_prefetch = [&](int j) {
#pragma unroll
        for (int u = 0; u < RPL; ++u) {
            const unsigned long long* p = rec_m + (size_t)j * rec_round + u * LPG;
            r0[u] = rec_load(p);
            r1[u] = rec_load(p + T);
        }
    };
    auto phase_b = [&](const float4 (&v)[NV], int j, int pb) {
        const int b = b0 + j * spr;
        settle(r0);
        settle(r1);
        // lane rj merges records rj, rj+LPG, ... of group rg in tile order,
        // then the group's LPG lanes a fixed xor tree (run by every lane, in
        // uniform control flow; lanes past the mergers carry zeros)
        const float ntile = (float)(Gm::TP * Gm::CPG4 * 4);
        float n = ntile, m = 0.0f, q = 0.0f;
        if (merger) {
#pragma unroll
            for (int u = 0; u < RPL; ++u) {
                const unsigned long long* p = rec_m + (size_t)j * rec_round + u * LPG;
                const float mj = rec_wait(p, r0[u], epoch, spin_limit, wf);
                const float qj = rec_wait(p + T, r1[u], epoch, spin_limit, wf);
                if (u == 0) {
                    m = mj;
                    q = qj;
                } else {
                    chan_merge(n, m, q, ntile, mj, qj);
                }
            }
        }
        // at level o each partial covers ntile * RPL * o values (a constant);
        // the group's total, HW * cpg, is a power of two, so q * inv_n is q / n.
        // A wave with no merging lane skips the tree (its values go unused);
        // the test is on scalars, so each wave runs the tree whole or not at
        // all.  Not with SHIFT: there the branch costs the loop vector-lane
        // spills of scalar registers.  Not without an activation: there the
        // loop is not short of vector issue, and the skip measured no gain.
        if (SHIFT || ACT == ACT_IDENTITY || wid_s * kWave < GT * LPG)
            for_xor_levels(lpg_scalar(LPG), [&](auto o) {
                xmerge_eq<decltype(o)::value>(m, q, ntile * (float)(RPL * decltype(o)::value));
            });
        if (merger && rj == 0) stat[pb][rg] = make_float2(m, rsqrtf(q * sh.inv_n + eps));
        lds_barrier();
        const float2 st = stat[pb][gl];
        const float mean = st.x, rs = st.y;
        if (t == 0 && tid < GT) {
            const float2 sg = stat[pb][tid];
            mu_out[b * sh.G + cb * GT + tid] = sg.x;
            rstd_out[b * sh.G + cb * GT + tid] = sg.y;
        }
        // gamma * (v - mean) * rs + beta = v * sc + sh0 per channel
        float4 sc, s0;
        sc.x = gm.x * rs;
        sc.y = gm.y * rs;
        sc.z = gm.z * rs;
        sc.w = gm.w * rs;
        s0.x = fmaf(-sc.x, mean, bt.x);
        s0.y = fmaf(-sc.y, mean, bt.y);
        s0.z = fmaf(-sc.z, mean, bt.z);
        s0.w = fmaf(-sc.w, mean, bt.w);
        float* ys = y + (size_t)b * sh.HW * sh.C + (size_t)(lrow + t * RC) * sh.C + c0;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float4 o;
            o.x = act_fwd<ACT>(fmaf(v[k].x, sc.x, s0.x));
            o.y = act_fwd<ACT>(fmaf(v[k].y, sc.y, s0.y));
            o.z = act_fwd<ACT>(fmaf(v[k].z, sc.z, s0.z));
            o.w = act_fwd<ACT>(fmaf(v[k].w, sc.w, s0.w));
            stS<NT>(ys + (size_t)(k * rstep_rows) * sh.C, o);
        }
    };

    // Round j: wait for stage buffer j % 2; take tile j into registers;
    // issue the loads of tile j + 2 into the same buffer; phase A on tile j;
    // phase B on tile j - 2 (in registers since round j - 2); prefetch the
    // records of tile j - 1, which phase B reads in the next round.  Two
    // tiles are in flight while a round computes, and a tile's records have
    // two rounds to arrive, so the exchange round trip (agent-scope store,
    // then load) stays off the critical path.  The register sets S0, S1, S2
    // hold tile j in S[j % 3]; the steady loop is unrolled by three so that
    // no tile is ever copied between registers.  Every round issues the same
    // vector-memory operations (loads past the last tile are issued against
    // an empty range) and the rounds without a phase B are peeled, so the
    // stage waits are constants:
    //   round 0: tile 1's NV loads were issued after tile 0's;
    //   round 1: round 0 issued NV loads;
    //   round 2: round 1 issued NV loads and 2 RPL record loads;
    //   round j >= 3: round j - 1 issued NV loads, NV stores, 2 RPL record loads;
    // plus, with SHIFT, the shift load issued before each tile's loads.
    if (w >= nt) return;
    const int K = (nt - w + P - 1) / P;
    float4 S0[NV], S1[NV], S2[NV];
    constexpr int SH = SHIFT ? 1 : 0;
    int pb = 0;
    auto steady_round = [&](int j, float4 (&cur)[NV], const float4 (&old)[NV]) {
        vm_wait<2 * NV + 2 * RPL + SH>();  // j >= 3
        take(cur, j);
        issue(j + 2, j & 1);
        phase_a(cur, j, pb);
        phase_b(old, j - 2, pb);
        records_prefetch(j - 1);
        pb ^= 1;
    };
    // gamma and beta are loaded right before the first two tiles' loads and
    // settled (so that their first use in the loop does not wait for the
    // staged tiles) only after those are issued: the tile loads no longer
    // wait for a round trip, and the settle waits for gamma and beta alone
    // (loads complete in order).
    gm = ld4(gamma + c0);
    bt = ld4(beta + c0);
    __builtin_amdgcn_sched_barrier(0);  // keep them above the tile loads
    issue(0, 0);
    issue(1, 1);
    settle(gm);
    settle(bt);
    vm_wait<NV + SH>();
    take(S0, 0);
    issue(2, 0);
    phase_a(S0, 0, pb);
    pb ^= 1;
    if (K > 1) {
        vm_wait<NV + SH>();
        take(S1, 1);
        issue(3, 1);
        phase_a(S1, 1, pb);
        records_prefetch(0);
        pb ^= 1;
        if (K > 2) {
            vm_wait<NV + 2 * RPL + SH>();
            take(S2, 2);
            issue(4, 0);
            phase_a(S2, 2, pb);
            phase_b(S0, 0, pb);
            records_prefetch(1);
            pb ^= 1;
            int j = 3;
            for (; j + 2 < K; j += 3) {
                steady_round(j, S0, S1);
                steady_round(j + 1, S1, S2);
                steady_round(j + 2, S2, S0);
            }
            if (j < K) steady_round(j, S0, S1);
            if (j + 1 < K) steady_round(j + 1, S1, S2);
        }
        // phase B of tiles K - 2 and K - 1, in S[(K - 2) % 3] and S[(K - 1) % 3]
        const int km = K % 3;
        if (km == 2) phase_b(S0, K - 2, pb);
        else if (km == 0) phase_b(S1, K - 2, pb);
        else phase_b(S2, K - 2, pb);
        pb ^= 1;
    }
    records_prefetch(K - 1);
    {
        const int km = K % 3;
        if (km == 1) phase_b(S0, K - 1, pb);
        else if (km == 2) phase_b(S1, K - 1, pb);
        else phase_b(S2, K - 1, pb);
    }
    vm_wait<0>();  // the loads past the last tile write the stage: let them land before the workgroup ends
    // the last active workgroup to finish advances the workspace's epoch
    __shared__ unsigned arrived;
    __syncthreads();
    if (tid == 0) {
        const unsigned active = (unsigned)(nt < P ? nt : P);
        arrived = __hip_atomic_fetch_add(wk.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == active - 1) {
            publish_epoch(wk, epoch);
            __hip_atomic_store(wk.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-arm
        }
    }
}

// ---------------------------------------------------------------------------
// Backward.  dy is the gradient of act(GN(x)); the pre-activation is
// recomputed from x, mu, rstd, gamma, beta.  Parks xhat and g = d*gamma.
// ---------------------------------------------------------------------------
// SHIFT: the input of the forward was x + shift[b, c]; besides dx the kernel
// writes, per tile, the column sums of dx over its pixel rows to colpart
// [tile][column block channel] (gns_colsum adds them per sample into the
// gradient of the shift).
template <class Gm, int ACT, int RPL, bool NT, bool SHIFT>
__global__ __launch_bounds__(Gm::TPB) void gns_bwd(float* __restrict__ dx, float* __restrict__ ggamma,
    float* __restrict__ gbeta, const float* __restrict__ dy,
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ mu, const float* __restrict__ rstd, const float* __restrict__ shift,
    float* __restrict__ colpart, Shape sh, Work wk, unsigned spin_limit) {
#pragma clang fp contract(fast)
    constexpr int NW = Gm::NW, NV = Gm::NV, GT = Gm::GT, TPB = Gm::TPB, CW4 = Gm::CW4;
    static_assert(NV == 2 && TPB * 16 == 16384, "stage slots (x then dy) as lds_take4 reads them");
    // Tile rows contiguous (one chunk of TP rows).  Measured against the
    // forward's interleaved rows at the north-star shape (same-box A/B): rows in
    // chunks of 16, 4, 2 and 1 gave 524, 535, 526 and 540 us against 508 us.
    constexpr int RC = Gm::TP;
    // Two stage buffers (x then dy of the tiles of the next two rounds,
    // direct-to-LDS loads); the tiles awaiting phase B (xhat, g) stay in
    // registers.
    __shared__ float4 stage[2][2 * NV * TPB];
    static_assert(2 * CW4 == kWave, "a wave's shift load covers the column block twice");
    __shared__ float4 shs[SHIFT ? 4 : 1][SHIFT ? kWave : 1];  // with SHIFT: the shift ring
    __shared__ float2 wred[2][GT][NW];          // (S1, S2) partials, laid out as in the forward
    __shared__ float2 stat[2][GT];              // group means of g and g * xhat
    __shared__ float cred[NW][CW4][8];          // per-wave dgamma/dbeta sums at the end (then the reducer's)
    // with SHIFT, during the tile loop: the per-wave column sums of a tile's
    // dx, double-buffered by the parity of the phase B that wrote them
    float4 (*csum)[NW][CW4] = reinterpret_cast<float4 (*)[NW][CW4]>(&cred[0][0][0]);
    static_assert(sizeof(float4) * 2 * NW * CW4 <= sizeof(cred), "column sums fit the reduction buffer");
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    // the wave index as a scalar: the direct-to-LDS loads take their LDS
    // address from a scalar register (M0), computed once per address
    const int wid_s = __builtin_amdgcn_readfirstlane(wid);
    const int col = lane % CW4, row0 = wid * Gm::RW + lane / CW4;
    const int gl = col / Gm::CPG4;
    const int P = gridDim.x, w = blockIdx.x;
    const int T = sh.T, NCB = sh.NCB;
    const int cb = (w / T) % NCB;
    const int t = w % T;
    const int c0 = cb * CW4 * 4 + col * 4;
    const int gglob = cb * GT + gl;             // global group index of this lane
    // The rows of a tile: RC consecutive rows at a time, tile t taking chunk t
    // of every T chunks.  The T tiles of a sample and column block partition
    // its rows for any RC, and the statistics merge over all of them; with
    // RC = 1 the tiles a team streams at once read neighbouring rows rather
    // than T separate blocks.
    static_assert(RC == Gm::TP || Gm::RSTEP % RC == 0, "row chunks");
    // local row r of tile t -> sample row (r / RC) T RC + t RC + r % RC
    const int lrow = (row0 / RC) * T * RC + row0 % RC;  // this lane's first row, tile 0
    constexpr bool kContig = RC == Gm::TP;
    const uint32_t voff = (uint32_t)(lrow * sh.C + c0) * 4u;
    const uint32_t rstep_rows = (uint32_t)(kContig ? Gm::RSTEP : Gm::RSTEP * T);
    const uint32_t rstep_bytes = rstep_rows * (uint32_t)sh.C * 4u;
    const uint32_t row_bytes = (uint32_t)sh.C * 4u;
    // gamma and beta of this lane's channels: held in registers (loaded once
    // the first tile's loads are out, at the tile loop's start), or, where
    // the tile loop needs those registers (the shift's column sums), read
    // from LDS in each phase A
    constexpr bool kAffineLds = SHIFT;
    __shared__ float4 affine[kAffineLds ? 2 : 1][kAffineLds ? CW4 : 1];
    float4 gm_r = make_float4(0.0f, 0.0f, 0.0f, 0.0f), bt_r = gm_r;
    if constexpr (kAffineLds) {
        if (tid < CW4) {
            affine[0][tid] = ld4(gamma + cb * CW4 * 4 + tid * 4);
            affine[1][tid] = ACT != ACT_IDENTITY ? ld4(beta + cb * CW4 * 4 + tid * 4) : gm_r;
        }
        __syncthreads();
    }
    // The launch's tag: its word is loaded here and used only from take_epoch
    // on, which the tile loop calls after the first tiles' loads are issued
    // (the scheduler would otherwise consume it right after the load and
    // hold those loads back by its round trip).
    unsigned ep_word = epoch_word(wk), epoch = 0u;
    unsigned long long tag = 0ull;
    auto take_epoch = [&]() {
        asm volatile("" : "+v"(ep_word));
        epoch = epoch_of(ep_word);
        tag = (unsigned long long)epoch << 32;
    };
    const WaitFail wf{wk.err, wk.hflag};
    // A spin limit of 0 lets no wait succeed: the launch flags itself as
    // timed out (the error path, forced from the host for its tests).
    if (spin_limit == 0 && blockIdx.x == 0 && threadIdx.x == 0) wait_failed(wf);
    const int LPG = T / RPL;
    const int rg = tid / LPG, rj = tid % LPG;
    const bool merger = rg < GT;
    const int nt = sh.ntiles;
    float4 cg = make_float4(0.0f, 0.0f, 0.0f, 0.0f), cbs = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    // Round j works on this workgroup's tile w + j * P (see the forward).
    const int b0 = w / (NCB * T), spr = P / (NCB * T);
    const int u0 = w / T, upr = P / T;
    auto real_of = [&](int j) { return w + j * P < nt; };
    // Record layout [unit][group][value][pixel tile]: the mergers of a group
    // read consecutive tiles, i.e. contiguous records.
    auto rec_slot = [&](int j, int g, int tt) { return wk.rec + ((size_t)((u0 + j * upr) * GT + g) * 2) * T + tt; };
    // The same addresses as per-lane bases plus a uniform step per round, so
    // the tile loop adds one scalar offset instead of redoing the index
    // arithmetic: the merging lane's first record (group rg, or GT - 1 past
    // the mergers; tile rj) and the group leader's own (group tid / NW; tile t).
    const size_t rec_round = (size_t)upr * GT * 2 * T;
    const unsigned long long* const rec_m = rec_slot(0, merger ? rg : GT - 1, rj);
    unsigned long long* const rec_s = rec_slot(0, tid / NW < GT ? tid / NW : GT - 1, t);
    // The x and dy loads of round j's tile into stage buffer sb (2 NV).  A
    // tile past the end is issued against an empty buffer range: the loads
    // read nothing and only keep the operation count of every round the same.
    // With SHIFT the forward's input was x + shift[b, c]: the shift ring as in
    // the forward, filled before each tile's x and dy loads.
    // One resource over the whole [B, C] shift for the kernel; the sample
    // moves the scalar offset (a tile past the end reads the last sample's).
    const __amdgpu_buffer_rsrc_t shr = sample_rsrc(shift, SHIFT ? (uint32_t)(sh.B * sh.C * 4) : 0u);
    const uint32_t shv = (uint32_t)(cb * CW4 * 4 + col * 4) * 4u;
    auto issue_shift = [&](int j) {
        if constexpr (SHIFT)
            dma16<false>(shr, &shs[j & 3][0], shv, (uint32_t)(real_of(j) ? b0 + j * spr : sh.B - 1) * row_bytes);
    };
    auto issue = [&](int j, int sb) {
        const bool real = real_of(j);
        const size_t so = (size_t)(real ? b0 + j * spr : 0) * sh.HW * sh.C;
        const uint32_t bytes = real ? sh.sample_bytes : 0u;
        const __amdgpu_buffer_rsrc_t rx = sample_rsrc(x + so, bytes);
        const __amdgpu_buffer_rsrc_t rd = sample_rsrc(dy + so, bytes);
        const uint32_t base = (uint32_t)(t * RC) * row_bytes;
        issue_shift(j);
#pragma unroll
        for (int k = 0; k < NV; ++k)
            dma16<NT>(rx, &stage[sb][k * TPB + wid_s * kWave], voff, base + (uint32_t)k * rstep_bytes);
#pragma unroll
        for (int k = 0; k < NV; ++k)
            dma16<NT>(rd, &stage[sb][(NV + k) * TPB + wid_s * kWave], voff, base + (uint32_t)k * rstep_bytes);
    };
    auto take = [&](float4 (&v)[2 * NV], int j) {
        if constexpr (SHIFT)
            lds_take4_shift<NV>(v, lds_addr(&stage[j & 1][tid]), lds_addr(&shs[j & 3][col]));
        else
            lds_take4(v, lds_addr(&stage[j & 1][tid]));
    };
    // Mean and rstd of this lane's group in round j's sample (two loads; a
    // tile past the end reads the last sample's and never uses them).
    float mean, rs;
    auto load_stats = [&](int j) {
        const int b = real_of(j) ? b0 + j * spr : sh.B - 1;
        mean = mu[b * sh.G + gglob];
        rs = rstd[b * sh.G + gglob];
    };
    // With SHIFT: the column sums of round j's tile (written by its phase B
    // into csum[par] after that phase's barrier) added over the waves in
    // order, one channel per lane, and stored to its row of colpart.  Called
    // past a later barrier and before the next phase B of the same parity
    // passes its own barrier, after which csum[par] is rewritten; the tile
    // loop calls it at the end of a round, where few registers are live.
    auto flush_colsum = [&](int j, int par) {
        if constexpr (SHIFT) {
            if (tid < CW4 * 4) {
                const float* cf = reinterpret_cast<const float*>(&csum[par][0][0]) + tid;
                float a = cf[0];
#pragma unroll 3
                for (int ww = 1; ww < NW; ++ww) a += cf[ww * CW4 * 4];
                colpart[(size_t)(w + j * P) * (CW4 * 4) + tid] = a;
            }
        } else {
            (void)j;
            (void)par;
        }
    };
    // phase A: v[0..NV) = x -> xhat, v[NV..2NV) = dy -> g in place; per-group
    // S1 = sum g, S2 = sum g*xhat -> records
    auto phase_a = [&](float4 (&v)[2 * NV], int j, int pb) {
        float4 s1v = make_float4(0.0f, 0.0f, 0.0f, 0.0f), s2v = s1v;
        const float4 gm = kAffineLds ? affine[0][col] : gm_r;
        const float4 bt = kAffineLds ? affine[1][col] : bt_r;
        const float nms = -mean * rs;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float4 xh, d;
            xh.x = fmaf(v[k].x, rs, nms);
            xh.y = fmaf(v[k].y, rs, nms);
            xh.z = fmaf(v[k].z, rs, nms);
            xh.w = fmaf(v[k].w, rs, nms);
            d = v[NV + k];
            if constexpr (ACT != ACT_IDENTITY) {
                d.x = d.x * act_grad<ACT>(fmaf(gm.x, xh.x, bt.x));
                d.y = d.y * act_grad<ACT>(fmaf(gm.y, xh.y, bt.y));
                d.z = d.z * act_grad<ACT>(fmaf(gm.z, xh.z, bt.z));
                d.w = d.w * act_grad<ACT>(fmaf(gm.w, xh.w, bt.w));
            }
            cg.x = fmaf(d.x, xh.x, cg.x);
            cg.y = fmaf(d.y, xh.y, cg.y);
            cg.z = fmaf(d.z, xh.z, cg.z);
            cg.w = fmaf(d.w, xh.w, cg.w);
            cbs.x += d.x;
            cbs.y += d.y;
            cbs.z += d.z;
            cbs.w += d.w;
            float4 g;
            g.x = d.x * gm.x;
            g.y = d.y * gm.y;
            g.z = d.z * gm.z;
            g.w = d.w * gm.w;
            s1v.x += g.x;
            s1v.y += g.y;
            s1v.z += g.z;
            s1v.w += g.w;
            s2v.x = fmaf(g.x, xh.x, s2v.x);
            s2v.y = fmaf(g.y, xh.y, s2v.y);
            s2v.z = fmaf(g.z, xh.z, s2v.z);
            s2v.w = fmaf(g.w, xh.w, s2v.w);
            v[k] = xh;
            v[NV + k] = g;
        }
        float s1 = (s1v.x + s1v.y) + (s1v.z + s1v.w);
        float s2 = (s2v.x + s2v.y) + (s2v.z + s2v.w);
        for_group_xor<Gm>([&](auto o) {
            xsum<decltype(o)::value>(s1);
            xsum<decltype(o)::value>(s2);
        });
        if (lane % CW4 % Gm::CPG4 == 0 && lane < CW4) wred[pb][gl][wave_slot<Gm>(gl, wid)] = make_float2(s1, s2);
        lds_barrier();
        // wave partials of group g summed on lanes (g, i) in a fixed xor tree
        static_assert(kWave % NW == 0 && GT * NW % kWave == 0, "a group's wave partials share a wave");
        if (tid < GT * NW) {  // whole waves: GT * NW is a multiple of 64
            const int g = tid / NW, i = tid % NW;
            const float2 ac = wred[pb][g][wave_slot<Gm>(g, i)];
            float a = ac.x, c = ac.y;
            for_xor_levels(NW, [&](auto o) {
                xsum<decltype(o)::value>(a);
                xsum<decltype(o)::value>(c);
            });
            if (i == 0) {
                unsigned long long* r = rec_s + (size_t)j * rec_round;
                rec_store(r, tagged(tag, a));
                rec_store(r + T, tagged(tag, c));
            }
        }
    };
    // Every lane loads (lanes past the mergers read group GT-1 and ignore it):
    // a branch here would put a path without these loads in front of the
    // record waits.
    unsigned long long r0[RPL] = {}, r1[RPL] = {};
    auto records_prefetch = [&](int j) {
#pragma unroll
        for (int u = 0; u < RPL; ++u) {
            const unsigned long long* p = rec_m + (size_t)j * rec_round + u * LPG;
            r0[u] = rec_load(p);
            r1[u] = rec_load(p + T);
        }
    };
    // phase B on a parked tile (xhat, g in v, its rstd rsv): merge its
    // records, form dx, store
    auto phase_b = [&](const float4 (&v)[2 * NV], float rsv, int j, int pb) {
        const int b = b0 + j * spr;
        settle(r0);
        settle(r1);
        // the group's LPG merging lanes add its records, then a fixed xor
        // tree (run by every lane, in uniform control flow; lanes past the
        // mergers carry zeros)
        float a = 0.0f, c = 0.0f;
        if (merger) {
#pragma unroll
            for (int u = 0; u < RPL; ++u) {
                const unsigned long long* p = rec_m + (size_t)j * rec_round + u * LPG;
                a += rec_wait(p, r0[u], epoch, spin_limit, wf);
                c += rec_wait(p + T, r1[u], epoch, spin_limit, wf);
            }
        }
        for_xor_levels(LPG, [&](auto o) {
            xsum<decltype(o)::value>(a);
            xsum<decltype(o)::value>(c);
        });
        if (merger && rj == 0) stat[pb][rg] = make_float2(a * sh.inv_n, c * sh.inv_n);
        lds_barrier();
        // dx = rs * ((g - m1) - xhat * m2) = g * rs + (xhat * (-rs m2) + (-rs m1))
        const float2 st = stat[pb][gl];
        const float a1 = -rsv * st.x, a2 = -rsv * st.y;
        float* dxs = dx + (size_t)b * sh.HW * sh.C + (size_t)(lrow + t * RC) * sh.C + c0;
        float4 cs = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const float4 xh = v[k];
            const float4 g = v[NV + k];
            float4 o;
            o.x = fmaf(g.x, rsv, fmaf(xh.x, a2, a1));
            o.y = fmaf(g.y, rsv, fmaf(xh.y, a2, a1));
            o.z = fmaf(g.z, rsv, fmaf(xh.z, a2, a1));
            o.w = fmaf(g.w, rsv, fmaf(xh.w, a2, a1));
            stS<NT>(dxs + (size_t)(k * rstep_rows) * sh.C, o);
            if constexpr (SHIFT) {
                cs.x += o.x;
                cs.y += o.y;
                cs.z += o.z;
                cs.w += o.w;
            }
        }
        if constexpr (SHIFT) {
            // this wave's rows of the tile, in a fixed xor tree over the row lanes
            static_assert(CW4 == 32, "one row level");
            xsum<32>(cs.x);
            xsum<32>(cs.y);
            xsum<32>(cs.z);
            xsum<32>(cs.w);
            if (lane < CW4) csum[pb][wid][lane] = cs;
        }
    };

    // Rounds as in the forward: round j waits for stage buffer j % 2, takes
    // tile j, issues tile j + 2's loads, runs phase A on tile j, loads tile
    // j + 1's statistics into the registers phase A has just used (a load
    // into a register that is then copied would make the copy wait for it),
    // runs phase B on tile j - 2 and prefetches tile j - 1's records.  The
    // backward keeps its tiles in v (tile j), pk1 (j - 1) and pk2 (j - 2) and
    // moves them along each round: unrolled by three as in the forward it
    // needs more than the 128 VGPRs a 1024-thread workgroup has and spills.
    // Stage waits (operations issued after the buffer's loads):
    //   round 0: tile 1's 2 NV loads;
    //   round 1: round 0's 2 NV tile loads and 2 statistics loads;
    //   round 2: round 1's 2 NV + 2 loads and 2 RPL record loads;
    //   round j >= 3: round j - 1's 2 NV + 2 loads, NV stores, 2 RPL record loads;
    // plus, with SHIFT, the shift load issued before each tile's loads.
    if (w < nt) {
        const int K = (nt - w + P - 1) / P;
        float4 v[2 * NV], pk1[2 * NV], pk2[2 * NV];
        float rs1 = 0.0f, rs2 = 0.0f;  // rstd of tiles j - 1 and j - 2
        constexpr int SH = SHIFT ? 1 : 0;  // the shift load issued before each tile's loads
        auto rotate = [&](float rs_j) {
#pragma unroll
            for (int k = 0; k < 2 * NV; ++k) {
                pk2[k] = pk1[k];
                pk1[k] = v[k];
            }
            rs2 = rs1;
            rs1 = rs_j;
        };
        int pb = 0;
        // round 0's statistics and (in registers) gamma and beta right before
        // the first two tiles' loads, settled after those are issued (see the
        // forward)
        load_stats(0);
        if constexpr (!kAffineLds) {
            gm_r = ld4(gamma + c0);
            if constexpr (ACT != ACT_IDENTITY) bt_r = ld4(beta + c0);
        }
        issue(0, 0);
        issue(1, 1);
        take_epoch();
        if constexpr (!kAffineLds) {
            settle(gm_r);
            settle(bt_r);
        }
        vm_wait<2 * NV + SH>();
        take(v, 0);
        issue(2, 0);
        phase_a(v, 0, pb);
        {
            const float rs_j = rs;
            load_stats(1);
            rotate(rs_j);
        }
        pb ^= 1;
        if (K > 1) {
            vm_wait<2 * NV + 2 + SH>();
            take(v, 1);
            issue(3, 1);
            phase_a(v, 1, pb);
            {
                const float rs_j = rs;
                load_stats(2);
                records_prefetch(0);
                rotate(rs_j);
            }
            pb ^= 1;
            if (K > 2) {
                vm_wait<2 * NV + 2 + 2 * RPL + SH>();
                take(v, 2);
                issue(4, 0);
                phase_a(v, 2, pb);
                {
                    const float rs_j = rs;
                    load_stats(3);
                    phase_b(pk2, rs2, 0, pb);
                    records_prefetch(1);
                    rotate(rs_j);
                }
                pb ^= 1;
                for (int j = 3; j < K; ++j) {
                    vm_wait<3 * NV + 2 + 2 * RPL + SH>();
                    take(v, j);
                    issue(j + 2, j & 1);
                    phase_a(v, j, pb);
                    const float rs_j = rs;
                    load_stats(j + 1);
                    phase_b(pk2, rs2, j - 2, pb);
                    records_prefetch(j - 1);
                    rotate(rs_j);
                    pb ^= 1;
                    flush_colsum(j - 3, pb);  // round j - 1's phase B, the other parity
                }
            }
            // tiles K - 2 and K - 1 (now pk2 and pk1)
            phase_b(pk2, rs2, K - 2, pb);
            if (K > 2) flush_colsum(K - 3, pb ^ 1);
            pb ^= 1;
        }
        records_prefetch(K - 1);
        phase_b(pk1, rs1, K - 1, pb);
        vm_wait<0>();  // the loads past the last tile write the stage: let them land before it is reused
        if constexpr (SHIFT) {  // the last two tiles, before the buffer serves the dgamma/dbeta sums
            __syncthreads();
            flush_colsum(K - 1, pb);
            if (K > 1) flush_colsum(K - 2, pb ^ 1);
            __syncthreads();
        }
    }

    if (w >= nt) take_epoch();

    // dgamma/dbeta partials of this workgroup: lanes with equal column own the
    // same 4 channels; sum over the wave's rows, then over the waves in order.
    float c8[8] = {cg.x, cg.y, cg.z, cg.w, cbs.x, cbs.y, cbs.z, cbs.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) xsum<32>(c8[j]);
    if (lane < CW4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) cred[wid][lane][j] = c8[j];
    }
    __syncthreads();
    // part[w][0 = dgamma, 1 = dbeta][channel within the column block], as
    // epoch-tagged records: the adders below accept exactly this launch's
    // values, so no fence orders them before the arrival count (an agent-scope
    // fence writes back the whole L2, which costs more than the wait).
    constexpr int NVAL = CW4 * 8;  // values per workgroup
    static_assert(TPB % NVAL == 0 && TPB / NVAL * NVAL <= NW * CW4 * 8, "team-sum layout");
    for (int i = tid; i < NVAL; i += TPB) {
        const int cl = i / 8, j = i % 8;
        float acc = cred[0][cl][j];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) acc += cred[ww][cl][j];
        rec_store(wk.part + (size_t)w * NVAL + (j >> 2) * (CW4 * 4) + cl * 4 + (j & 3), tagged(tag, acc));
    }
    __shared__ unsigned arrived;
    const int team = w / T;
    __syncthreads();
    if (tid == 0) arrived = __hip_atomic_fetch_add(wk.count + 1 + team, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != (unsigned)T - 1) return;

    // Last member of the team: add the T partials in member order (Q
    // interleaved chains, then the chains in order).  Every partial was
    // stored before its workgroup arrived, so each wait is short.
    constexpr int Q = TPB / NVAL;
    float(*chain)[NVAL] = reinterpret_cast<float(*)[NVAL]>(&cred[0][0][0]);
    {
        const int v = tid % NVAL, q = tid / NVAL;  // q is uniform over the wave (NVAL >= 64)
        const unsigned long long* src = wk.part + ((size_t)team * T + q) * NVAL + v;
        chain[q][v] = rec_sum<16>(src, (size_t)Q * NVAL, (T - q + Q - 1) / Q, epoch, spin_limit, wf);
    }
    __syncthreads();
    for (int v = tid; v < NVAL; v += TPB) {
        float acc = chain[0][v];
#pragma unroll
        for (int q = 1; q < Q; ++q) acc += chain[q][v];
        rec_store(wk.tpart + (size_t)team * NVAL + v, tagged(tag, acc));
    }
    __syncthreads();
    if (tid == 0) {
        __hip_atomic_store(wk.count + 1 + team, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-arm
        arrived = __hip_atomic_fetch_add(wk.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const int nteams = P / T;
    if (arrived != (unsigned)nteams - 1) return;

    // Last team: dgamma/dbeta of channel c = the sums of the teams of its
    // column block (team k owns column block k mod NCB), in team order.
    for (int i = tid; i < 2 * sh.C; i += TPB) {
        const int d = i / sh.C, c = i % sh.C;
        const int cbc = c / (CW4 * 4), cl = c % (CW4 * 4);
        const unsigned long long* p = wk.tpart + (size_t)cbc * NVAL + d * (CW4 * 4) + cl;
        (d ? gbeta : ggamma)[c] = rec_sum<4>(p, (size_t)NCB * NVAL, (nteams - cbc + NCB - 1) / NCB, epoch,
                                             spin_limit, wf);
    }
    if (tid == 0) {
        publish_epoch(wk, epoch);  // every workgroup has arrived, so all have read the old one
        __hip_atomic_store(wk.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace gns
}  // namespace nnk

// ---------------------------------------------------------------------------
// Host side (k_gns_fwd.hip / k_gns_bwd.hip).
// ---------------------------------------------------------------------------
// Streaming geometry: 1024 threads, tiles of 32 float4 columns (128
// channels); forward tiles of 128 pixel rows (64 KB), backward of 64 (32 KB of
// x and 32 KB of dy): the staged and the parked tile fill 128 KB of the
// workgroup's LDS either way.  Measured alternative: forward tiles of whole
// 256-channel rows (64 float4 columns x 64 rows, teams of 64) ran 411 us
// against 372 us at the north-star shape.
namespace nnk {
namespace gns {
constexpr int kTpb = 1024;
constexpr int kFwdCw4 = 32;
constexpr int kBwdCw4 = 32;
constexpr int kFwdTp = 128;
constexpr int kBwdTp = 64;
constexpr int kMaxGrid = 1024;        // persistent workgroups at most
// Polls of one record before a wait gives up (each poll sleeps and reloads,
// ~1 us): far beyond any wait of a correct launch, which is bounded by the
// run time of the grid itself.
constexpr unsigned kSpinLimit = 1u << 20;

// Kernel keys of the persistent-grid cache (nnk_gns_grid): forwards below
// kGnsBwdKeys, backwards from it.
constexpr int kGnsBwdKeys = 256;

struct Plan {
    bool ok;
    int cpg4, rpl;
    Shape sh;
    size_t ws_floats;        // workspace needed (header + records [+ partials])
    size_t rec_offset;       // in bytes from the workspace start
    size_t part_offset;
    size_t tpart_offset;
    size_t colpart_offset;   // backward with a shift: per-tile column sums of dx (plain floats)
    size_t ws_shift_floats;  // workspace needed by the backward with a shift
};

// Applicability and sizes; `bwd` selects the backward geometry.
Plan make_plan(bool bwd, int B, int HW, int C, int G);
}  // namespace gns
}  // namespace nnk

// Launch the streaming kernels when the shape fits and the device can hold
// the persistent grid; return false (nothing launched) otherwise.  `ws` is a
// device workspace of at least plan.ws_floats floats whose records region
// never holds this launch's epoch and whose counters are zero (a zero-filled
// workspace, only ever used by these launchers, is both).
// With `shift` non-null the input is x + shift[b, c] (formed in registers;
// x is not modified), and the backward also writes gshift[b, c] = the sum over
// the pixels of dx (its workspace then needs plan.ws_shift_floats floats).
bool nnk_gns_forward(int act, float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, const float* shift, int B, int HW, int C, int G, float eps, float* ws, hipStream_t s);
bool nnk_gns_backward(int act, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, const float* shift, float* gshift,
    int B, int HW, int C, int G, float* ws, hipStream_t s);
// Whether nnk_gns_forward / nnk_gns_backward have a kernel for a shift on this
// shape and activation (the grid's fit on the device aside).
bool nnk_gns_shift_forward_shape_ok(int act, int B, int HW, int C, int G);
bool nnk_gns_shift_backward_shape_ok(int act, int B, int HW, int C, int G);
