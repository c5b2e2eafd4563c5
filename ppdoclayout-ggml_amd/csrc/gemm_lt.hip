// Shape-fitted GEMM on v_mfma_f32_16x16x4f32 for dense k-major operands (1x1
// convs, F(4,3) plane products): C[m][n] = epi(sum_k A[k][m] B[k][n]).
//
// One block of 4 waves owns an MTM x MTN output tile and walks the whole K
// range: no split-K pass, no partial tiles in memory.  The tile menu is wide
// (32 x 160, 128 x 96, 96 x 32, ...) so that the planner can pick a shape
// whose tile count is just under a multiple of the CU count; with 16 x 16
// matrix blocks a wave tile only has to be a multiple of 16 on each side.
//
// Pipeline per k tile of DU rows: the global loads of the tile after next
// are issued into one register set, the current tile's fragments are read
// from LDS into the matrix pipe, then the other register set (the next tile,
// loaded one step earlier) goes to the other LDS buffer and one block barrier
// closes the step (two LDS buffers, two register stages).  With KG = 2 the
// block runs 8 waves, two per SIMD: group g contracts the second or first
// half of each tile's k rows, and the two partial tiles are added through
// LDS before the epilogue.  LDS
// rows are padded to a stride of 16 (mod 32) floats: the four k rows that a
// fragment read touches (lanes 0-15, 16-31, 32-47, 48-63) fall on disjoint
// banks.
//
// 16x16x4 operand layout: lane l supplies A[m0 + l%16][k0 + l/16] and
// B[k0 + l/16][n0 + l%16]; result register r of lane l is row 4*(l/16) + r,
// column l%16.
//
// Edges: columns past M (resp. the float4-readable width of B) are clamped to
// the last whole float4 (they only feed discarded outputs); rows past K are
// zeroed in the registers before they reach LDS.
//
// Persistent blocks: the grid holds at most kLtMaxBlocks blocks; each XCD
// owns a contiguous range of tiles (blocks sharing operand panels share an
// L2) and its blocks stride through that range.
#include <algorithm>
#include <cstdlib>
#include <string>
#include <utility>

#include "device_math.h"
#include "ppdl_internal.h"

namespace ppdl {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4g(const float *p) { return *reinterpret_cast<const float4 *>(p); }
// v, or zeros when !ok (per component: a select of the whole float4 would be
// lowered through scratch memory)
__device__ __forceinline__ float4 keep_if(float4 v, bool ok) {
    return make_float4(ok ? v.x : 0.0f, ok ? v.y : 0.0f, ok ? v.z : 0.0f, ok ? v.w : 0.0f);
}

template <int MTM, int MTN, int DU, int WGM, int KG>
__global__ __launch_bounds__(256 * KG) void k_gemm_lt(GemmArgs g, int tiles_m, int tiles_mn) {
    constexpr int NT = 256 * KG;
    constexpr int WGN = 4 / WGM, WM = MTM / WGM, WN = MTN / WGN, FM = WM / 16, FN = WN / 16;
    static_assert(WGM * WGN == 4 && WM % 16 == 0 && WN % 16 == 0, "wave tile");
    constexpr int PA = MTM + (48 - MTM % 32) % 32, PB = MTN + (48 - MTN % 32) % 32;  // = 16 (mod 32)
    constexpr int QA = MTM / 4, QB = MTN / 4;                                          // float4 per k row
    constexpr int LA = DU * QA / NT, LB = DU * QB / NT;                                // copies per thread
    static_assert(LA * NT == DU * QA && LB * NT == DU * QB && LA >= 1 && LB >= 1, "whole copies");
    constexpr int QM = FM / 4, QN = FN / 4;  // runs of four interleaved 16-wide blocks
    constexpr int SG = DU / 4 / KG;          // k steps per group and tile
    static_assert(SG >= 1 && SG * KG * 4 == DU, "k steps per group");
    constexpr int SA = DU * PA, SB = DU * PB;  // floats per LDS stage
    static_assert(KG == 1 || 4 * 64 * FM * FN * 4 <= 2 * (SA + SB), "group reduction space");
    __shared__ __attribute__((aligned(16))) float smem[2 * (SA + SB)];
    float *const As = smem, *const Bs = smem + 2 * SA;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = wave >> 2, wq = wave & 3;  // k group; position in the 2-d wave grid
    const int l16 = lane & 15, kq = lane >> 4;
    const int wm0 = (wq % WGM) * WM, wn0 = (wq / WGM) * WN;
    const int M = g.M, N = g.N, K = g.K;
    const int lda = (int)g.lda, ldb = (int)g.ldb;
    const int nk = (K + DU - 1) / DU;
    // wave-relative row of row x of block i, column of column x of block j
    auto row_of = [](int i, int x) { return i < 4 * QM ? 64 * (i >> 2) + 4 * x + (i & 3) : 64 * QM + 16 * (i - 4 * QM) + x; };
    auto col_of = [](int j, int x) { return j < 4 * QN ? 64 * (j >> 2) + 4 * x + (j & 3) : 64 * QN + 16 * (j - 4 * QN) + x; };

    // this XCD's tile range and this block's slot in it
    const int T = tiles_mn * g.batch;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per = (int)(gridDim.x >> 3) + ((int)(gridDim.x & 7) > xcd);
    const int q = T >> 3, rr = T & 7;
    const int t_begin = xcd * q + min(xcd, rr), t_end = t_begin + q + (xcd < rr ? 1 : 0);

    // copy e of this thread: tile row and LDS column (global column per tile)
    int ar[LA], acl[LA], br[LB], bcl[LB];
#pragma unroll
    for (int e = 0; e < LA; e++) {
        const int idx = e * NT + tid;
        ar[e] = idx / QA;
        acl[e] = 4 * (idx % QA);
    }
#pragma unroll
    for (int e = 0; e < LB; e++) {
        const int idx = e * NT + tid;
        br[e] = idx / QB;
        bcl[e] = 4 * (idx % QB);
    }

    for (int tile = t_begin + slot; tile < t_end; tile += per) {
        const int bz = tile / tiles_mn;
        const int t = tile - bz * tiles_mn;
        const int m0 = (t % tiles_m) * MTM, n0 = (t / tiles_m) * MTN;
        const float *__restrict__ A = g.A + (int64_t)bz * g.sA;
        const float *__restrict__ B = g.B + (int64_t)bz * g.sB;
        int ac[LA], bc[LB];
#pragma unroll
        for (int e = 0; e < LA; e++) ac[e] = min(m0 + acl[e], M - 4);
#pragma unroll
        for (int e = 0; e < LB; e++) bc[e] = min(n0 + bcl[e], g.n_vec - 4);

        // two register stages: tile kt + 2 is in flight while tile kt + 1 goes
        // from registers to LDS
        float4 ra0[LA], rb0[LB], ra1[LA], rb1[LB];
        auto gload = [&](float4 (&ra)[LA], float4 (&rb)[LB], int kt) {
            const int k0 = kt * DU;
#pragma unroll
            for (int e = 0; e < LA; e++) ra[e] = ld4g(A + (uint32_t)(min(k0 + ar[e], K - 1) * lda + ac[e]));
#pragma unroll
            for (int e = 0; e < LB; e++) rb[e] = ld4g(B + (uint32_t)(min(k0 + br[e], K - 1) * ldb + bc[e]));
        };
        // copies [e0, e1) of the LA + LB copies (A first) of tile kt into LDS buffer buf
        auto spart = [&](int buf, const float4 (&ra)[LA], const float4 (&rb)[LB], int kt, int e0, int e1) {
            const int k0 = kt * DU;
#pragma unroll
            for (int e = 0; e < LA; e++)
                if (e >= e0 && e < e1)
                    *reinterpret_cast<float4 *>(As + buf * SA + ar[e] * PA + acl[e]) = keep_if(ra[e], k0 + ar[e] < K);
#pragma unroll
            for (int e = 0; e < LB; e++)
                if (LA + e >= e0 && LA + e < e1)
                    *reinterpret_cast<float4 *>(Bs + buf * SB + br[e] * PB + bcl[e]) = keep_if(rb[e], k0 + br[e] < K);
        };
        auto sstore = [&](int buf, const float4 (&ra)[LA], const float4 (&rb)[LB], int kt) {
            const int k0 = kt * DU;
#pragma unroll
            for (int e = 0; e < LA; e++)
                *reinterpret_cast<float4 *>(As + buf * SA + ar[e] * PA + acl[e]) = keep_if(ra[e], k0 + ar[e] < K);
#pragma unroll
            for (int e = 0; e < LB; e++)
                *reinterpret_cast<float4 *>(Bs + buf * SB + br[e] * PB + bcl[e]) = keep_if(rb[e], k0 + br[e] < K);
        };

        f32x4 acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // this group's SG k steps of a tile, fragments one step ahead of the
        // MFMAs.  Each run of four 16-wide blocks interleaves its columns
        // (block 4q + u, column c <-> wave column 64q + 4c + u), so a lane's
        // operands of the four blocks are adjacent: one 16-byte LDS read.
        auto compute = [&](int buf, auto &&after_step) {
            const float *as = As + buf * SA + wm0, *bs = Bs + buf * SB + wn0;
            float a[2][FM], b[2][FN];
            auto rd = [&](int ks, float (&aa)[FM], float (&bb)[FN]) {
                const int kk = 4 * (grp * SG + ks) + kq;
#pragma unroll
                for (int qq = 0; qq < QM; qq++) {
                    const float4 v = *reinterpret_cast<const float4 *>(as + kk * PA + 64 * qq + 4 * l16);
                    aa[4 * qq] = v.x, aa[4 * qq + 1] = v.y, aa[4 * qq + 2] = v.z, aa[4 * qq + 3] = v.w;
                }
#pragma unroll
                for (int i = 4 * QM; i < FM; i++) aa[i] = as[kk * PA + 64 * QM + 16 * (i - 4 * QM) + l16];
#pragma unroll
                for (int qq = 0; qq < QN; qq++) {
                    const float4 v = *reinterpret_cast<const float4 *>(bs + kk * PB + 64 * qq + 4 * l16);
                    bb[4 * qq] = v.x, bb[4 * qq + 1] = v.y, bb[4 * qq + 2] = v.z, bb[4 * qq + 3] = v.w;
                }
#pragma unroll
                for (int j = 4 * QN; j < FN; j++) bb[j] = bs[kk * PB + 64 * QN + 16 * (j - 4 * QN) + l16];
            };
            rd(0, a[0], b[0]);
#pragma unroll
            for (int ks = 0; ks < SG; ks++) {
                // the next step's reads go out before this step's MFMAs, into
                // their own registers (left to itself the scheduler sinks them
                // below the MFMAs and reuses the registers: a full LDS round
                // trip per step)
                if (ks + 1 < SG) rd(ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ks & 1][i], b[ks & 1][j], acc[i][j], 0, 0,
                                                                         0);
                after_step(ks);
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // per-row bias of this lane's output rows, loaded under the k loop
        float rbias[FM][4];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) rbias[i][r] = g.bias ? g.bias[min(m0 + wm0 + row_of(i, 4 * kq + r), M - 1)] : 0.0f;

        gload(ra0, rb0, 0);
        gload(ra1, rb1, min(1, nk - 1));
        sstore(0, ra0, rb0, 0);
        __syncthreads();
        // two k tiles per trip (buffer 0 then 1); every step loads and stores
        // a tile (past the end: tile nk - 1 again, into the idle buffer), so
        // no condition surrounds the staging registers
        constexpr int NC = LA + LB;  // copies per thread and tile
        for (int kt = 0; kt < nk; kt += 2) {
            const int t1 = min(kt + 1, nk - 1), t2 = min(kt + 2, nk - 1);
            gload(ra0, rb0, t2);
            __builtin_amdgcn_sched_barrier(0);
            compute(0, [&](int ks) { spart(1, ra1, rb1, t1, ks * NC / SG, (ks + 1) * NC / SG); });
            __syncthreads();
            if (kt + 1 >= nk) break;
            gload(ra1, rb1, min(kt + 3, nk - 1));
            __builtin_amdgcn_sched_barrier(0);
            compute(1, [&](int ks) { spart(0, ra0, rb0, t2, ks * NC / SG, (ks + 1) * NC / SG); });
            __syncthreads();
        }

        if constexpr (KG == 2) {
            // group 1 hands its partial tile to group 0 through the idle LDS
            float *red = smem + wq * (64 * FM * FN * 4) + lane;
            if (grp == 1) {
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) red[((i * FN + j) * 4 + r) * 64] = acc[i][j][r];
            }
            __syncthreads();
            if (grp == 0) {
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[i][j][r] += red[((i * FN + j) * 4 + r) * 64];
            }
        }

        if (grp == 0) {
            float *__restrict__ C = g.C + (int64_t)bz * g.sC;
            const float *__restrict__ Ad = g.add ? g.add + (int64_t)bz * g.sC : nullptr;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    const int n = n0 + wn0 + col_of(j, l16);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = m0 + wm0 + row_of(i, 4 * kq + r);
                        if (m < M && n < N) {
                            const int64_t idx = (int64_t)m * g.ldc + n;
                            float v = acc[i][j][r];
                            if (g.bias) v += rbias[i][r];
                            if (g.add_mode == 1) v += Ad[idx];
                            v = act_f(v, g.act);
                            if (g.add_mode == 2) v += Ad[idx];
                            else if (g.add_mode == 3) v = refine_box(v, Ad[idx]);
                            C[idx] = v;
                        }
                    }
                }
        }
        if constexpr (KG == 2) __syncthreads();  // the reduction space is the next tile's stage 0
    }
}

struct LtCfg {
    int mtm, mtn, du, wgm, kg;
};
// The tile menu: (MTM, MTN, DU, waves along M, k groups)
constexpr LtCfg kLt[] = {
    {32, 160, 64, 2, 2},   // 0: wave 16 x 80
    {32, 96, 64, 2, 2},    // 1: wave 16 x 48
    {128, 96, 32, 2, 1},   // 2: wave 64 x 48, one group
    {96, 32, 64, 2, 2},    // 3: wave 48 x 16
    {32, 64, 64, 2, 2},    // 4: wave 16 x 32
    {64, 64, 32, 2, 2},    // 5: wave 32 x 32
    {128, 64, 32, 2, 2},   // 6: wave 64 x 32
    {64, 128, 32, 2, 2},   // 7: wave 32 x 64
    {32, 128, 64, 2, 2},   // 8: wave 16 x 64
    {32, 160, 64, 2, 1},   // 9: wave 16 x 80, one group
    {32, 128, 32, 2, 1},   // 10: wave 16 x 64, one group
    {64, 32, 64, 2, 2},    // 11: wave 32 x 16
};
constexpr int kNumLt = sizeof(kLt) / sizeof(kLt[0]);
constexpr int kLtMaxBlocks = 2048;

template <int C>
hipError_t launch_cfg(const GemmArgs &g, hipStream_t s) {
    constexpr LtCfg c = kLt[C];
    const int tiles_m = (g.M + c.mtm - 1) / c.mtm, tiles_n = (g.N + c.mtn - 1) / c.mtn;
    const int64_t T = (int64_t)tiles_m * tiles_n * g.batch;
    if (T <= 0 || T > 0x7fffffff) return hipErrorInvalidValue;
    // grid: every tile its own block up to the cap, rounded to whole XCD rows
    int64_t grid = std::min<int64_t>(T, kLtMaxBlocks);
    grid = (grid + 7) / 8 * 8;
    hipLaunchKernelGGL((k_gemm_lt<c.mtm, c.mtn, c.du, c.wgm, c.kg>), dim3((unsigned)grid), dim3(256 * c.kg), 0, s, g,
                       tiles_m, tiles_m * tiles_n);
    return hipGetLastError();
}

template <int... I>
hipError_t launch_any(int cfg, const GemmArgs &g, hipStream_t s, std::integer_sequence<int, I...>) {
    hipError_t r = hipErrorInvalidValue;
    ((cfg == I ? (r = launch_cfg<I>(g, s), 0) : 0), ...);
    return r;
}

}  // namespace

int gemm_lt_num_cfgs() { return kNumLt; }

// dense k-major A and B with 4-aligned extents and 16-byte aligned bases;
// 32-bit element offsets within one batch plane; a CHW result (no
// transposed store, no per-column bias, no sign-bit output)
bool gemm_lt_ok(const GemmArgs &g) {
    const auto a16 = [](const void *p) { return (((uintptr_t)p) & 15) == 0; };
    return !g.a_rowmajor && !g.bits && !g.a_add && !g.a_w4 && !g.c_trans && !g.bias_n && g.M >= 4 && g.M % 4 == 0 &&
           g.n_vec >= 4 &&
           g.K >= 1 && g.lda % 4 == 0 && g.ldb % 4 == 0 && g.sA % 4 == 0 && g.sB % 4 == 0 && a16(g.A) && a16(g.B) &&
           (int64_t)g.K * g.lda + g.M < 0x7fffffff && (int64_t)g.K * g.ldb + g.n_vec < 0x7fffffff && g.batch >= 1;
}

hipError_t gemm_lt(const GemmArgs &g, int cfg, hipStream_t s) {
    if (cfg < 0 || cfg >= kNumLt || !gemm_lt_ok(g)) return hipErrorInvalidValue;
    return launch_any(cfg, g, s, std::make_integer_sequence<int, kNumLt>{});
}

std::string gemm_lt_name(int cfg) {
    if (cfg < 0 || cfg >= kNumLt) return "";
    const LtCfg &c = kLt[cfg];
    return "k_gemm_lt<" + std::to_string(c.mtm) + ", " + std::to_string(c.mtn) + ", " + std::to_string(c.du) + ", " +
           std::to_string(c.wgm) + ", " + std::to_string(c.kg) + ">";
}

// The menu entry with the least estimated time, or -1 (the caller's other
// kernels).  Opt-in: PPDL_LT unset or "off": never; "auto": the estimate
// where the caller `wants` this kernel for the shape (unless PPDL_GEMM_TILE
// pins a plan of the other kernels); "<index>": that entry whenever the
// operands allow (sweeps, tests).  Read per call.  Estimate: rounds of
// resident tiles (one block per CU) x per-tile time, where a tile's k step
// costs max(matrix work, operand fetch) on one CU.
//
// Why opt-in: on the split-K 1x1 convs of the network it is faster per
// launch (in-graph kernel traces: enc_in1 44 -> 28 us with the reduction
// launch it removes, stage-3 agg1 62 -> 46 us), yet the whole graph replayed
// 2.7 us slower with it than without (two graphs in one process, replayed
// alternately, 8 rounds of 100; A/A spread +-1 us).
int gemm_lt_pick(const GemmArgs &g, int cus, bool wanted) {
    const char *e = getenv("PPDL_LT");
    if (!e || !*e || e[0] == 'o' || !gemm_lt_ok(g)) return -1;
    if (e[0] != 'a') {
        const int c = atoi(e);
        return c >= 0 && c < kNumLt ? c : -1;
    }
    const char *pin = getenv("PPDL_GEMM_TILE");
    if (!wanted || (pin && *pin)) return -1;
    if (cus <= 0) cus = 256;
    int best = -1;
    double best_t = 0.0;
    for (int c = 0; c < kNumLt; c++) {
        const LtCfg &t = kLt[c];
        const int64_t tiles = (int64_t)((g.M + t.mtm - 1) / t.mtm) * ((g.N + t.mtn - 1) / t.mtn) * g.batch;
        const int64_t rounds = (tiles + cus - 1) / cus;
        const double mma = (double)t.mtm * t.mtn / 128.0;      // cycles per k on one CU
        const double feed = (double)(t.mtm + t.mtn) / 16.0;    // 64 B per cycle from L2
        const double step = std::max(mma, feed);
        const double tt = (double)rounds * (g.K * step + 2000.0);
        if (best < 0 || tt < best_t) {
            best = c;
            best_t = tt;
        }
    }
    return best;
}

}  // namespace ppdl
