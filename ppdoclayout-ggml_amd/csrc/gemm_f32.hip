// Strict-FP32 GEMM core on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32).
//
//   C[m][n] = act( sum_k At[k][m] * B[k][n] + bias[m] )
//
// One kernel serves every conv GEMM of the tagged-op path:
//   * 1x1 conv (op 3 / 14):   At = wr[ic][oc], B = x[ic][pixel], C = CHW out;
//   * F(4,3) madd (op 12):    36 planes on the batch axis, At = wg4[p][ic][oc],
//                             B = dt[p][ic][tile], C = yt[p][oc][tile];
//   * k2 / k3-s2 conv (16):   At = wr[tap][ic][oc], B = an implicit im2col view
//                             of the CHW input (no column buffer in HBM).
// Every operand is k-major, so both global loads and C stores are coalesced
// along the fastest axis (m for At, n for B and C).
//
// Tiling: a 256-thread block = 4 wave64s owns a BM x BN tile of C; each wave
// owns WM x WN = (32*TM) x (32*TN) of it as TM*TN 32x32 MFMA accumulators
// (16 fp32 per lane each).  K advances 16 at a time through a double-buffered
// LDS stage: the next tile's global loads are in flight while the MFMAs of
// the current one issue.  Inside a 16-deep k tile, lanes 0-31 supply k rows
// 0..7 and lanes 32-63 rows 8..15 to the 8 MFMAs (each MFMA contracts 2 k),
// which keeps every LDS read a row-contiguous 32-float run (no bank conflict
// with the +4 row pad).  No TF32/bf16 emulation anywhere: the products and
// the accumulation are IEEE fp32 inside the matrix core.
#include "ppdl_internal.h"

namespace ppdl {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 16;

__device__ __forceinline__ float act_f(float v, int act) {
    if (act == 1) return v > 0.0f ? v : 0.0f;
    if (act == 2) return v / (1.0f + expf(-v));
    return v;
}

// Blocks are dispatched round-robin over the 8 XCDs (hardware id % 8).  Give
// each XCD a contiguous range of logical tiles so that tiles sharing operands
// (same n columns, same batch plane) hit the same L2.
__device__ __forceinline__ int xcd_remap(int hw, int n) {
    const int q = n >> 3, r = n & 7;
    const int xcd = hw & 7, slot = hw >> 3;
    return xcd * q + (xcd < r ? xcd : r) + slot;
}

template <int BM, int BN, int WGM, bool IM2COL>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmArgs g, int tiles_m, int tiles_mn) {
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int PA = BM + 4, PB = BN + 4;
    constexpr int EA = kBK * BM / kThreads, EB = kBK * BN / kThreads;
    constexpr int RA = kThreads / BM, RB = kThreads / BN;
    static_assert(TM >= 1 && TN >= 1 && EA >= 1 && EB >= 1, "bad tile");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");

    __shared__ float As[2][kBK][PA];
    __shared__ float Bs[2][kBK][PB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bz = logical / tiles_mn;
    const int t = logical - bz * tiles_mn;
    const int tm = t % tiles_m, tn = t / tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const float *__restrict__ A = g.A + (int64_t)bz * g.sA;
    const float *__restrict__ B = g.B + (int64_t)bz * g.sB;
    float *__restrict__ C = g.C + (int64_t)bz * g.sC;
    const int M = g.M, N = g.N, K = g.K;

    // loader coordinates: each thread owns one m column of the A tile and one
    // n column of the B tile, and walks k rows RA / RB apart
    const int am = tid % BM, ak = tid / BM;
    const int bn = tid % BN, bk = tid / BN;
    const int gm = m0 + am, gn = n0 + bn;
    const bool am_ok = gm < M, bn_ok = gn < N;
    int iy0 = 0, ix0 = 0;
    if (IM2COL) {
        const int oy = gn / g.OW, ox = gn - oy * g.OW;
        iy0 = oy * g.S - g.P;
        ix0 = ox * g.S - g.P;
    }
    const int64_t plane = (int64_t)g.IH * g.IW;

    float ra[EA], rb[EB];
    auto load = [&](int k0) {
#pragma unroll
        for (int e = 0; e < EA; e++) {
            const int k = k0 + ak + e * RA;
            ra[e] = (am_ok && k < K) ? A[(int64_t)k * g.lda + gm] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < EB; e++) {
            const int k = k0 + bk + e * RB;
            float v = 0.0f;
            if (bn_ok && k < K) {
                if (IM2COL) {
                    const int tap = k / g.IC, ic = k - tap * g.IC;
                    const int kh = tap / g.KW, kw = tap - kh * g.KW;
                    const int iy = iy0 + kh, ix = ix0 + kw;
                    if (iy >= 0 && iy < g.IH && ix >= 0 && ix < g.IW)
                        v = B[ic * plane + (int64_t)iy * g.IW + ix];
                } else {
                    v = B[(int64_t)k * g.ldb + gn];
                }
            }
            rb[e] = v;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int e = 0; e < EA; e++) As[buf][ak + e * RA][am] = ra[e];
#pragma unroll
        for (int e = 0; e < EB; e++) Bs[buf][bk + e * RB][bn] = rb[e];
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int wm0 = (wave % WGM) * WM, wn0 = (wave / WGM) * WN;
    const int l32 = lane & 31, lk = (lane >> 5) * (kBK / 2);
    const int nk = (K + kBK - 1) / kBK;

    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK / 2; kk++) {
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = As[cur][lk + kk][wm0 + i * 32 + l32];
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = Bs[cur][lk + kk][wn0 + j * 32 + l32];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }

    // epilogue: 32x32 accumulator layout — lane owns column (lane & 31) and
    // rows 8*(r/4) + 4*(lane/32) + r%4 of register r
    const float *__restrict__ bias = g.bias;
    const int act = g.act;
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn0 + j * 32 + l32;
        if (n < N) {
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < M) {
                        float v = acc[i][j][r];
                        if (bias) v += bias[m];
                        C[(int64_t)m * g.ldc + n] = act_f(v, act);
                    }
                }
            }
        }
    }
}

struct TileCfg {
    int bm, bn, wgm;
};
// Candidate block shapes (BM, BN, waves along M).  Wave tiles range from
// 64x64 (4 accumulators) down to 32x32.
constexpr TileCfg kCfgs[] = {
    {128, 128, 2},  // wave 64x64
    {64, 128, 2},   // wave 32x64
    {128, 64, 2},   // wave 64x32
    {64, 64, 2},    // wave 32x32
    {32, 256, 1},   // wave 32x64
    {32, 128, 1},   // wave 32x32
};
constexpr int kNumSimd = 256 * 4;  // MI355X: 256 CUs x 4 SIMDs

// Pick the block shape that minimises the MFMA time of the busiest SIMD:
// rounds(wave tiles / SIMDs) x MFMAs per wave tile, plus the padding waste of
// partial tiles.  Ties go to the larger tile (less LDS and L2 traffic).
int pick_cfg(int M, int N, int batch) {
    int best = 0;
    double best_cost = 1e300;
    for (int c = 0; c < (int)(sizeof(kCfgs) / sizeof(kCfgs[0])); c++) {
        const TileCfg &t = kCfgs[c];
        const int64_t tiles = (int64_t)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
        const int64_t waves = tiles * 4;
        const int64_t rounds = (waves + kNumSimd - 1) / kNumSimd;
        const int tm = t.bm / t.wgm / 32, tn = t.bn / (4 / t.wgm) / 32;
        const double cost = (double)rounds * tm * tn * (1.0 + 0.02 * (4.0 / (tm * tn)));
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = c;
        }
    }
    return best;
}

template <int BM, int BN, int WGM, bool IM2COL>
hipError_t launch(const GemmArgs &g, hipStream_t s) {
    const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
    const int64_t total = (int64_t)tiles_m * tiles_n * g.batch;
    if (total <= 0 || total > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm<BM, BN, WGM, IM2COL>), dim3((unsigned)total), dim3(kThreads), 0, s,
                       g, tiles_m, tiles_m * tiles_n);
    return hipGetLastError();
}

template <bool IM2COL>
hipError_t dispatch(const GemmArgs &g, hipStream_t s) {
    switch (pick_cfg(g.M, g.N, g.batch)) {
        case 0: return launch<128, 128, 2, IM2COL>(g, s);
        case 1: return launch<64, 128, 2, IM2COL>(g, s);
        case 2: return launch<128, 64, 2, IM2COL>(g, s);
        case 3: return launch<64, 64, 2, IM2COL>(g, s);
        case 4: return launch<32, 256, 1, IM2COL>(g, s);
        default: return launch<32, 128, 1, IM2COL>(g, s);
    }
}

}  // namespace

hipError_t gemm_dense(const GemmArgs &g, hipStream_t s) { return dispatch<false>(g, s); }
hipError_t gemm_im2col(const GemmArgs &g, hipStream_t s) { return dispatch<true>(g, s); }

}  // namespace ppdl
