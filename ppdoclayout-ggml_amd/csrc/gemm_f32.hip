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
// Every operand is k-major, so global loads and C stores are contiguous along
// the fastest axis (m for At, n for B and C).
//
// Tiling: a 256-thread block = 4 wave64s owns a BM x BN tile of C; each wave
// owns (32*TM) x (32*TN) of it as TM*TN 32x32 MFMA accumulators.  K advances
// BK = 32 at a time through a double-buffered LDS stage fed by a two-deep
// register prefetch: while the MFMAs of k tile t issue, tile t+1 waits in
// registers for its LDS slot and tile t+2's global loads are in flight, so a
// load has two tiles of MFMA work to hide behind.  Inside a k tile, lanes
// 0-31 feed k rows 0..15 and lanes 32-63 rows 16..31 to the 16 MFMA steps
// (each MFMA contracts 2 k); all fragments of a tile are read from LDS before
// its MFMAs issue, so LDS latency overlaps the matrix pipe.
//
// Split-K (optional, for long-K shapes with few output tiles): S blocks share
// one output tile, each contracting a contiguous range of k tiles and storing
// its fp32 partial tile to a caller-provided workspace; a second small kernel
// sums the S partials in fixed order s = 0..S-1 and applies bias/act.  The
// kernel boundary orders the two, so no block waits on or fences for another,
// and the result does not depend on scheduling.
//
// No TF32/bf16 emulation anywhere: products and accumulation are IEEE fp32 in
// the matrix core; split partials are summed in fp32.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "device_math.h"

namespace ppdl {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 32;

__device__ __forceinline__ float4 ld4(const float *p) {
    float4 v;
    __builtin_memcpy(&v, p, 16);  // dword-aligned dwordx4 load
    return v;
}

struct SplitArgs {
    int splits;  // S (1 = no split)
    int ktiles_per_split;
    float *partials;  // S x batch x M x N
    // block order: 1 = split-major (logical block = split * tiles + tile), so
    // each XCD's contiguous range of blocks covers about 1/8 of the (split,
    // tile) space and fetches one k range of A and B instead of every m row
    // of A; 0 = tile-major (the S splits of a tile adjacent)
    int split_major;
};

// (split, tile) of logical block `logical` of a split launch over `tiles`
// output tiles
__device__ __forceinline__ void split_of(const SplitArgs &sp, int logical, int tiles, int *split, int *tile) {
    if (sp.split_major) {
        *split = logical / tiles;
        *tile = logical - *split * tiles;
    } else {
        *split = logical % sp.splits;
        *tile = logical / sp.splits;
    }
}

// Per-thread staging registers for one k tile.
template <int EA, int EB4, int EB1>
struct Stage {
    float4 a[EA];
    float4 b4[EB4];
    float b1[EB1];
    uint32_t ok1;  // im2col: bit e set when element e is inside the image
};

// Epilogue of a wave's (32 TM) x (32 TN) accumulator tile whose top-left
// output is (mw, nw): split-K partials, or bias / residual add / act and the
// store in C's layout.  32x32 accumulator layout: lane owns column (lane & 31)
// and rows 8*(r/4) + 4*(lane/32) + r%4 of register r.  Only registers
// r in [RB, RB + RN) are stored (RB, RN multiples of 4).
//
// A per-row bias (bias_n == 0) may come pre-loaded in registers (PB, from
// load_row_bias before the k loop, so its load latency hides under the
// MFMAs): bv[i][r - RB] is the bias of row m of register r of tile row i.
template <int TM, int RN>
struct RowBias {
    float v[TM][RN];
};

// rows of registers rb .. rb + RN - 1 (rb a multiple of 4; register rb + r
// holds the row of register r plus 2 * rb)
template <int TM, int RN>
__device__ __forceinline__ void load_row_bias(RowBias<TM, RN> &bv, const GemmArgs &g, int mw, int rb, int lane) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < RN; r++) {
            const int m = mw + 2 * rb + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            bv.v[i][r] = g.bias[min(m, g.M - 1)];
        }
}

template <int TM, int TN, bool SPLIT, int RB = 0, int RN = 16, bool PB = false>
__device__ __forceinline__ void gemm_epilogue(const f32x16 (&acc)[TM][TN], const GemmArgs &g, const SplitArgs &sp,
                                              int split, int bz, int mw, int nw, int lane,
                                              const RowBias<TM, RN> *bv = nullptr) {
    const int M = g.M, N = g.N, l32 = lane & 31;
    if (SPLIT) {
        float *__restrict__ P = sp.partials + ((int64_t)split * g.batch + bz) * M * N;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = nw + j * 32 + l32;
            if (n < N) {
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int r = RB; r < RB + RN; r++) {
                        const int m = mw + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        if (m < M) P[(int64_t)m * N + n] = acc[i][j][r];
                    }
            }
        }
        return;
    }

    if (g.bits) {
        // sign bits of the products: a half-wave holds 32 consecutive n of one
        // row (the launch checks N % 32 == 0), so one ballot per register
        // yields row m's word (lanes 0-31) and row m + 4's (lanes 32-63)
        const int nwords = N >> 5;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n0 = nw + j * 32;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = RB; r < RB + RN; r++) {
                    const unsigned long long b = __ballot(acc[i][j][r] > 0.0f);
                    const int m = mw + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if ((lane & 31) == 0 && m < M && n0 < N)
                        g.bits[(int64_t)bz * M * nwords + (int64_t)m * nwords + (n0 >> 5)] =
                            (uint32_t)(lane ? (b >> 32) : b);
                }
        }
        return;
    }
    const float *__restrict__ bias = g.bias;
    const int act = g.act, add_mode = g.add_mode, bias_n = g.bias_n;
    float *__restrict__ C = g.C + (int64_t)bz * g.sC;
    const float *__restrict__ Ad = g.add ? g.add + (int64_t)bz * g.sC : nullptr;
    // bias of (m, n) for tile row i, register r (PB: the pre-loaded value)
    auto bias_of = [&](int i, int r, int m, int n) -> float {
        if (PB && !bias_n) return bv->v[i][r - RB];
        return bias[bias_n ? n : m];
    };
    auto epi = [&](float v, float bval, int64_t idx) {
        if (bias) v += bval;
        if (add_mode == 1) v += Ad[idx];
        v = act_f(v, act);
        if (add_mode == 2) v += Ad[idx];
        else if (add_mode == 3) v = refine_box(v, Ad[idx]);
        return v;
    };
    if (!g.c_trans) {
        // the store loop once per common activation (none, ReLU, SiLU), so
        // the unrolled loop a launch runs carries one activation's code
        auto store = [&](auto actc) {
            constexpr int A = decltype(actc)::value;
            auto epa = [&](float v, float bval, int64_t idx) {
                if (bias) v += bval;
                if (add_mode == 1) v += Ad[idx];
                v = act_t<A>(v, act);
                if (add_mode == 2) v += Ad[idx];
                else if (add_mode == 3) v = refine_box(v, Ad[idx]);
                return v;
            };
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = nw + j * 32 + l32;
                if (n < N) {
#pragma unroll
                    for (int i = 0; i < TM; i++) {
#pragma unroll
                        for (int r = RB; r < RB + RN; r++) {
                            const int m = mw + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                            if (m < M) {
                                const int64_t idx = (int64_t)m * g.ldc + n;
                                C[idx] = epa(acc[i][j][r], bias ? bias_of(i, r, m, n) : 0.0f, idx);
                            }
                        }
                    }
                }
            }
        };
        if (act == kActNone) store(std::integral_constant<int, kActNone>{});
        else if (act == kActRelu) store(std::integral_constant<int, kActRelu>{});
        else if (act == kActSilu) store(std::integral_constant<int, kActSilu>{});
        else store(std::integral_constant<int, -1>{});
    } else {
        // C[n][m]: registers 4g..4g+3 hold 4 consecutive m of one n
        const bool vec_ok = (g.ldc % 4 == 0) && ((((uintptr_t)C) & 15) == 0) &&
                            (!Ad || ((((uintptr_t)Ad) & 15) == 0));
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = nw + j * 32 + l32;
            if (n < N) {
#pragma unroll
                for (int i = 0; i < TM; i++) {
#pragma unroll
                    for (int q = RB / 4; q < (RB + RN) / 4; q++) {
                        const int mb = mw + i * 32 + 8 * q + 4 * (lane >> 5);
                        const int64_t idx = (int64_t)n * g.ldc + mb;
                        if (vec_ok && mb + 3 < M) {
                            float4 v;
                            v.x = epi(acc[i][j][4 * q + 0], bias ? bias_of(i, 4 * q + 0, mb + 0, n) : 0.0f, idx + 0);
                            v.y = epi(acc[i][j][4 * q + 1], bias ? bias_of(i, 4 * q + 1, mb + 1, n) : 0.0f, idx + 1);
                            v.z = epi(acc[i][j][4 * q + 2], bias ? bias_of(i, 4 * q + 2, mb + 2, n) : 0.0f, idx + 2);
                            v.w = epi(acc[i][j][4 * q + 3], bias ? bias_of(i, 4 * q + 3, mb + 3, n) : 0.0f, idx + 3);
                            *reinterpret_cast<float4 *>(C + idx) = v;
                        } else {
#pragma unroll
                            for (int u = 0; u < 4; u++)
                                if (mb + u < M)
                                    C[idx + u] = epi(acc[i][j][4 * q + u], bias ? bias_of(i, 4 * q + u, mb + u, n) : 0.0f,
                                                     idx + u);
                        }
                    }
                }
            }
        }
    }
}

// AMODE 0: A k-major; AMODE 1: A row-major (K % 4 == 0, lda % 4 == 0).
// BMODE 0: dense B; BMODE 1: implicit im2col B (generic, or one kernel tap
// per k tile when IC % kBK == 0); BMODE 2: implicit im2col B with IC >= kBK
// or IC == kBK / 2, at most two taps per k tile (its own instantiation: its
// loader needs more registers than BMODE 1's).
template <int BM, int BN, int WGM, int AMODE, int BMODE, bool SPLIT>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmArgs g, SplitArgs sp, int tiles_m, int tiles_mn) {
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int PA = BM + 4, PB = BN + 4;
    // A k-major: float4 along m, BM/4 threads per k row.  A row-major:
    // float4 along k, kBK/4 threads per m row, 32 rows per pass.
    constexpr int TA = BM / 4, RA = kThreads / TA, EA = AMODE == 0 ? kBK / RA : BM / (kThreads / (kBK / 4));
    // B dense: float4 along n; B im2col: one column per thread
    constexpr int TB4 = BN / 4, RB4 = kThreads / TB4, EB4 = BMODE == 0 ? kBK / RB4 : 1;
    constexpr int RB1 = kThreads / BN, EB1 = BMODE >= 1 ? kBK / RB1 : 1;
    constexpr int KH = kBK / 2;  // MFMA k-steps per tile
    static_assert(TM >= 1 && TN >= 1 && EA >= 1 && EB4 >= 1 && EB1 >= 1, "bad tile");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    using St = Stage<EA, EB4, EB1>;

    __shared__ __attribute__((aligned(16))) float As[2][kBK][PA];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBK][PB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    int split = 0, tile_id = logical;
    if (SPLIT) split_of(sp, logical, tiles_mn * g.batch, &split, &tile_id);
    const int bz = tile_id / tiles_mn;
    const int t = tile_id - bz * tiles_mn;
    const int tm = t % tiles_m, tn = t / tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = g.M, N = g.N, K = g.K;

    const int nk_total = (K + kBK - 1) / kBK;
    const int kt0 = SPLIT ? split * sp.ktiles_per_split : 0;
    const int kt1 = SPLIT ? min(nk_total, kt0 + sp.ktiles_per_split) : nk_total;
    const int nk = kt1 - kt0;

    const float *__restrict__ A = g.A + (int64_t)bz * g.sA;
    const float *__restrict__ B = g.B + (int64_t)bz * g.sB;

    // ---- loader state ----
    const int am = (tid % TA) * 4, ak = tid / TA;  // A k-major
    const int gm = m0 + am;
    const int ak4 = (tid % (kBK / 4)) * 4, amr = tid / (kBK / 4);  // A row-major
    constexpr int RA1 = kThreads / (kBK / 4);
    const int bn4 = (tid % TB4) * 4, bk4 = tid / TB4;  // dense B
    const int gn4 = n0 + bn4;
    const int bn1 = tid % BN, bk1 = tid / BN;  // im2col B
    const int gn1 = n0 + bn1;
    const bool bn_ok = gn1 < N;
    int iy0 = 0, ix0 = 0;
    if (BMODE >= 1) {
        const int oy = gn1 / g.OW, ox = gn1 - oy * g.OW;
        iy0 = oy * g.S - g.P;
        ix0 = ox * g.S - g.P;
    }
    // operand extents per batch plane fit in int32 (checked on the host)
    const int plane = g.IH * g.IW;
    // last float4 start of a B row: N - 4, or the padded width - 4 when B's
    // rows have room for whole float4s past N (columns nobody stores)
    const int nclamp = (g.n_vec > 0 ? g.n_vec : N) - 4;
    const int lda = (int)g.lda, ldb = (int)g.ldb;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int wm0 = (wave % WGM) * WM, wn0 = (wave / WGM) * WN;
    const int l32 = lane & 31, lk = (lane >> 5) * KH;

    // One k tile = KH MFMA steps, taken in pairs: a pair's A and B fragments
    // are two adjacent k rows (one ds_read2 per 32-wide strip).  Fragments
    // are read two pairs ahead of the MFMAs that use them, and the schedule
    // is pinned (sched_group_barrier) so each pair's reads issue behind the
    // previous pair's MFMAs: LDS latency hides under the matrix pipe even
    // with a single wave per SIMD.
    constexpr int NP = KH / 2;
    auto compute = [&](int buf) {
        float2 fa[NP][TM], fb[NP][TN];
        auto rd = [&](int p) {
#pragma unroll
            for (int i = 0; i < TM; i++) {
                fa[p][i].x = As[buf][lk + 2 * p][wm0 + i * 32 + l32];
                fa[p][i].y = As[buf][lk + 2 * p + 1][wm0 + i * 32 + l32];
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                fb[p][j].x = Bs[buf][lk + 2 * p][wn0 + j * 32 + l32];
                fb[p][j].y = Bs[buf][lk + 2 * p + 1][wn0 + j * 32 + l32];
            }
        };
        rd(0);
        rd(1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * (TM + TN), 0);
#pragma unroll
        for (int p = 0; p < NP; p++) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[p][i].x, fb[p][j].x, acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[p][i].y, fb[p][j].y, acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * TM * TN, 0);
            if (p + 2 < NP) {
                rd(p + 2);
                __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
            }
        }
    };

    // The loads only issue (clamped, always-valid addresses); every mask is
    // applied when the stage is written to LDS.  That keeps a fixed number of
    // loads per stage with no use of their results before the store, so the
    // compiler waits for one stage while the next stays in flight.  The
    // edge/interior choice is made once per block (EDGE).  Float4 loads are
    // used unless the tile crosses an M or N edge that is not a multiple of 4:
    // with a 4-aligned edge a float4 is either wholly inside or wholly past
    // it, and one past it is clamped to the last valid float4 (finite values
    // in rows / columns the epilogue never stores).  Other edge tiles load
    // clamped scalars.
    auto body = [&](auto edge_tag, auto tap_tag) {
        constexpr bool EDGE = decltype(edge_tag)::value;
        // im2col k tiles: 1 = one tap per tile (IC % kBK == 0, K % kBK == 0),
        // 2 = at most two taps (IC >= kBK), 0 = generic
        constexpr int TAPS = decltype(tap_tag)::value;
        auto load = [&](St &r, int kt) {
            const int k0 = kt * kBK;
            if (AMODE == 0) {
#pragma unroll
                for (int e = 0; e < EA; e++) {
                    const int k = min(k0 + ak + e * RA, K - 1);
                    const float *row = A + (uint32_t)(k * lda);
                    if (!EDGE) {
                        r.a[e] = ld4(row + min(gm, M - 4));
                    } else {
                        r.a[e].x = row[min(gm + 0, M - 1)];
                        r.a[e].y = row[min(gm + 1, M - 1)];
                        r.a[e].z = row[min(gm + 2, M - 1)];
                        r.a[e].w = row[min(gm + 3, M - 1)];
                    }
                }
            } else {
                // rows clamped into [0, M), k chunks into [0, K): K % 4 == 0,
                // so a chunk is entirely inside or outside
                const int k = min(k0 + ak4, K - 4);
#pragma unroll
                for (int e = 0; e < EA; e++) {
                    const int m = min(m0 + amr + e * RA1, M - 1);
                    r.a[e] = ld4(A + (uint32_t)(m * lda + k));
                }
            }
            if (BMODE == 0) {
#pragma unroll
                for (int e = 0; e < EB4; e++) {
                    const int k = min(k0 + bk4 + e * RB4, K - 1);
                    const float *row = B + (uint32_t)(k * ldb);
                    if (!EDGE) {
                        r.b4[e] = ld4(row + min(gn4, nclamp));
                    } else {
                        r.b4[e].x = row[min(gn4 + 0, N - 1)];
                        r.b4[e].y = row[min(gn4 + 1, N - 1)];
                        r.b4[e].z = row[min(gn4 + 2, N - 1)];
                        r.b4[e].w = row[min(gn4 + 3, N - 1)];
                    }
                }
            } else if (TAPS == 1) {
                // the whole k tile is one tap: one bounds test and base per
                // tile, rows RB1 channels apart.  A lane outside the image reads
                // a clamped in-image address (its value is masked at the store),
                // not one shared address.
                const int tap = k0 / g.IC;
                const int kh = tap / g.KW, kw = tap - kh * g.KW;
                const int iy = iy0 + kh, ix = ix0 + kw;
                const bool ok = bn_ok && iy >= 0 && iy < g.IH && ix >= 0 && ix < g.IW;
                const uint32_t base = (uint32_t)((k0 - tap * g.IC + bk1) * plane +
                                                 min(max(iy, 0), g.IH - 1) * g.IW + min(max(ix, 0), g.IW - 1));
#pragma unroll
                for (int e = 0; e < EB1; e++) r.b1[e] = B[base + (uint32_t)(e * RB1 * plane)];
                r.ok1 = ok ? 0xFFFFFFFFu : 0u;
            } else if (TAPS == 2) {
                // IC >= kBK, or IC == kBK / 2 (k tiles start on tap
                // boundaries): a k tile spans at most two kernel taps, so each
                // row picks one of two per-tile bases and bounds tests; rows
                // are RB1 channels apart.  A lane outside the image reads a
                // clamped in-image address (its value is masked at the store).
                const int tap0 = k0 / g.IC, ic0 = k0 - tap0 * g.IC;
                const int ntap = g.K / g.IC;
                uint32_t base[2];
                bool okt[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int tap = min(tap0 + h, ntap - 1);
                    const int kh = tap / g.KW, kw = tap - kh * g.KW;
                    const int iy = iy0 + kh, ix = ix0 + kw;
                    okt[h] = bn_ok && tap0 + h < ntap && iy >= 0 && iy < g.IH && ix >= 0 && ix < g.IW;
                    // channel of row r: ic0 + r (tap0) or ic0 + r - IC (tap0 + 1)
                    base[h] = (uint32_t)((ic0 - h * g.IC) * plane + min(max(iy, 0), g.IH - 1) * g.IW +
                                         min(max(ix, 0), g.IW - 1));
                }
                const int split = g.IC - ic0;  // rows r < split are tap0's
                uint32_t okm = 0;
#pragma unroll
                for (int e = 0; e < EB1; e++) {
                    const int rr = bk1 + e * RB1;
                    const bool second = rr >= split;
                    r.b1[e] = B[(second ? base[1] : base[0]) + (uint32_t)(rr * plane)];
                    okm |= ((second ? okt[1] : okt[0]) && k0 + rr < K ? 1u : 0u) << e;
                }
                r.ok1 = okm;
            } else {
                // k = (kh*KW + kw)*IC + ic: decompose the first row once, then
                // step ic by RB1 with carries into kw and kh
                int k = k0 + bk1;
                int tap = k / g.IC;
                int ic = k - tap * g.IC;
                int kh = tap / g.KW;
                int kw = tap - kh * g.KW;
                uint32_t okm = 0;
#pragma unroll
                for (int e = 0; e < EB1; e++) {
                    const int iy = iy0 + kh, ix = ix0 + kw;
                    const bool ok = bn_ok && k < K && iy >= 0 && iy < g.IH && ix >= 0 && ix < g.IW;
                    r.b1[e] = B[ok ? (uint32_t)(ic * plane + iy * g.IW + ix) : 0u];
                    okm |= (ok ? 1u : 0u) << e;
                    k += RB1;
                    ic += RB1;
                    while (ic >= g.IC) {
                        ic -= g.IC;
                        if (++kw == g.KW) {
                            kw = 0;
                            ++kh;
                        }
                    }
                }
                r.ok1 = okm;
            }
        };
        auto store = [&](const St &r, int buf, int kt) {
            const int k0 = kt * kBK;
            if (AMODE == 0) {
#pragma unroll
                for (int e = 0; e < EA; e++) {
                    float4 v = r.a[e];
                    const bool kin = k0 + ak + e * RA < K;
                    v.x = (kin && (!EDGE || gm + 0 < M)) ? v.x : 0.0f;
                    v.y = (kin && (!EDGE || gm + 1 < M)) ? v.y : 0.0f;
                    v.z = (kin && (!EDGE || gm + 2 < M)) ? v.z : 0.0f;
                    v.w = (kin && (!EDGE || gm + 3 < M)) ? v.w : 0.0f;
                    *reinterpret_cast<float4 *>(&As[buf][ak + e * RA][am]) = v;
                }
            } else {
                const bool kin = k0 + ak4 < K;
#pragma unroll
                for (int e = 0; e < EA; e++) {
                    const int mr = amr + e * RA1;
                    const bool ok = kin && m0 + mr < M;
                    As[buf][ak4 + 0][mr] = ok ? r.a[e].x : 0.0f;
                    As[buf][ak4 + 1][mr] = ok ? r.a[e].y : 0.0f;
                    As[buf][ak4 + 2][mr] = ok ? r.a[e].z : 0.0f;
                    As[buf][ak4 + 3][mr] = ok ? r.a[e].w : 0.0f;
                }
            }
            if (BMODE == 0) {
#pragma unroll
                for (int e = 0; e < EB4; e++) {
                    float4 v = r.b4[e];
                    const bool kin = k0 + bk4 + e * RB4 < K;
                    v.x = (kin && (!EDGE || gn4 + 0 < N)) ? v.x : 0.0f;
                    v.y = (kin && (!EDGE || gn4 + 1 < N)) ? v.y : 0.0f;
                    v.z = (kin && (!EDGE || gn4 + 2 < N)) ? v.z : 0.0f;
                    v.w = (kin && (!EDGE || gn4 + 3 < N)) ? v.w : 0.0f;
                    *reinterpret_cast<float4 *>(&Bs[buf][bk4 + e * RB4][bn4]) = v;
                }
            } else {
#pragma unroll
                for (int e = 0; e < EB1; e++) Bs[buf][bk1 + e * RB1][bn1] = ((r.ok1 >> e) & 1u) ? r.b1[e] : 0.0f;
            }
        };

        // Two-deep pipeline: r0/r1 alternate as the staging registers of even
        // / odd k tiles, LDS buffer 0/1 likewise.  A trip takes two tiles and
        // has no exit in the middle (an exit there leaves a path on which the
        // prefetch is still in flight at the loop head, and every trip then
        // drains it); an odd last tile is computed after the loop.  Loads and
        // stores past the last tile repeat the last tile (clamped), so every
        // trip issues the same instructions; those stages are never read.
        if (nk <= 0) return;  // an empty split range contributes zeros
        const int klast = kt1 - 1;
        St r0, r1;
        load(r0, kt0);
        store(r0, 0, kt0);
        load(r1, min(kt0 + 1, klast));
        __syncthreads();
        int it = 0;
        for (; it + 1 < nk; it += 2) {
            load(r0, min(kt0 + it + 2, klast));
            // keep the prefetch ahead of the MFMAs (sunk below them, its
            // destination registers get recycled as fragment registers)
            __builtin_amdgcn_sched_barrier(0);
            compute(0);
            __builtin_amdgcn_sched_barrier(0);
            store(r1, 1, kt0 + it + 1);
            __syncthreads();
            load(r1, min(kt0 + it + 3, klast));
            __builtin_amdgcn_sched_barrier(0);
            compute(1);
            __builtin_amdgcn_sched_barrier(0);
            store(r0, 0, min(kt0 + it + 2, klast));
            __syncthreads();
        }
        if (it < nk) compute(0);
    };
    const bool edge_m = AMODE == 0 && m0 + BM > M && (M & 3) != 0;  // row-major A clamps rows itself
    const bool edge_n = BMODE == 0 && n0 + BN > N && g.n_vec == 0;  // im2col B masks per element
    if constexpr (BMODE == 1) {
        using T0 = std::integral_constant<int, 0>;
        using T1 = std::integral_constant<int, 1>;
        const bool one = g.IC % kBK == 0 && K % kBK == 0;
        if (edge_m || edge_n) {
            if (one) body(std::true_type{}, T1{});
            else body(std::true_type{}, T0{});
        } else {
            if (one) body(std::false_type{}, T1{});
            else body(std::false_type{}, T0{});
        }
    } else if constexpr (BMODE == 2) {
        using T2 = std::integral_constant<int, 2>;
        if (edge_m || edge_n) body(std::true_type{}, T2{});
        else body(std::false_type{}, T2{});
    } else {
        using T0 = std::integral_constant<int, 0>;
        if (edge_m || edge_n) body(std::true_type{}, T0{});
        else body(std::false_type{}, T0{});
    }

    gemm_epilogue<TM, TN, SPLIT>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS variant for dense k-major A and B (1x1 convs, F(4,3) planes)
// whose M, N, lda, ldb are multiples of 4 with 16-byte aligned bases.  Each
// wave moves its share of a k tile with global_load_lds_dwordx4 (16 bytes per
// lane into m0 + 16 * lane): no staging registers, no LDS store instructions,
// and the next tile's copy is in flight while the current one is consumed.
// The LDS tile is [k][m] (resp. [k][n]) unpadded, 4 rows of 64 floats or 8
// of 32 per wave instruction.
//
// The copy is issued through inline asm: the compiler's own LDS-DMA tracking
// cannot tell the stages apart and would drain every copy before any LDS
// read.  Ordering is explicit instead: s_waitcnt vmcnt for this wave's copies
// of the tile, then the block barrier for everyone else's.
//
// Edges: rows past K and columns past M / n_vec are clamped to valid
// addresses (values that only reach discarded outputs); on the global last k
// tile, A rows at or past K are zeroed in LDS before use.
typedef __attribute__((address_space(3))) float lds_f32;
__device__ __forceinline__ uint32_t lds_off(float *p) { return (uint32_t)(uintptr_t)(lds_f32 *)p; }
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved: nothing else in these kernels uses it
__device__ __forceinline__ void dma16(const float *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((((N >> 4) & 3) << 14) | (0xF << 8) | (0x7 << 4) | (N & 0xF));
}

// global_load_lds_dwordx4 with a wave-uniform 64-bit base (SGPR pair) and a
// 32-bit per-lane byte offset
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved: nothing else in these kernels uses it
__device__ __forceinline__ void dma16s(uint64_t base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
#pragma clang diagnostic pop
// (readfirstlane returns int: each half goes through uint32_t, else the low
// half would sign-extend into the high one)
__device__ __forceinline__ uint64_t uniform_ptr(const float *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    return ((uint64_t)hi << 32) | lo;
}

// NS LDS stages: NS - 1 tiles in flight while one is computed.  KG wave
// groups: KG = 2 runs 8 waves per block, group g contracting the k rows
// [16g, 16g + 16) of every tile, and sums the two partial tiles through LDS
// before the epilogue (twice the waves per SIMD for the same tile count).
// One loop body per k tile (the stage is a runtime index): a body duplicated
// per stage let the compiler move the accumulators between register files at
// every tile.  A wave reads all of its fragments of a tile before the tile's
// MFMAs, so the chain waits for LDS once per tile.
//
// TAIL (64x64, KG = 2, no split): balances the last round of tiles.  Each XCD
// holds a contiguous range of cnt tiles on its `cus` CUs; when the remainder
// r = cnt mod cus is at most cus / 2, the last r tiles of the range run as 2r
// half tiles (32 columns each), so the CUs that take a third (fourth, ...)
// block take half a tile's work.  A half tile's work goes to waves 0-3 (one
// per SIMD: two 32-row positions x the two k groups); waves 4-7 only share
// the copies.  Blocks past an XCD's count exit at once.
template <int BM, int BN, int WGM, bool SPLIT, int NS, int KG, bool TAIL = false>
__global__ __launch_bounds__(kThreads * KG) void k_gemm_dma(GemmArgs g, SplitArgs sp, int tiles_m, int tiles_mn,
                                                            int cus) {
    static_assert(NS >= 2 && NS <= 4 && (KG == 1 || KG == 2), "stages / groups");
    static_assert(!TAIL || (BM == 64 && BN == 64 && WGM == 2 && KG == 2 && !SPLIT), "tail layout");
    constexpr int NT = kThreads * KG;
    constexpr int WGN = 4 / WGM, WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
    constexpr int IA = kBK * BM / 4 / NT, IB = kBK * BN / 4 / NT;  // copies per wave per tile
    constexpr int KH = kBK / 2, KQ = KH / KG;                       // k rows per half-wave and group
    static_assert(IA >= 1 && IB >= 1 && TM >= 1 && TN >= 1, "bad tile");
    constexpr int SA = kBK * BM, SB = kBK * BN;  // stage sizes (floats)
    __shared__ __attribute__((aligned(1024))) float smem[NS * (SA + SB)];
    float *const As = smem, *const Bs = smem + NS * SA;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int grp = wave >> 2, wq = wave & 3;  // k group, position in the 2-d wave grid
    int logical, half = -1;              // half: which 32 columns of a half tile
    if constexpr (TAIL) {
        const int T = tiles_mn * g.batch;
        const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
        const int q = T >> 3, rr = T & 7;
        const int cnt = q + (xcd < rr ? 1 : 0), start = xcd * q + min(xcd, rr);
        const int r = cnt % cus;
        const int h = (r > 0 && 2 * r <= cus) ? r : 0;
        const int nfull = cnt - h;
        if (slot >= cnt + h) return;  // the whole block, before any barrier
        if (slot < nfull) {
            logical = start + slot;
        } else {
            const int j = slot - nfull;
            logical = start + nfull + (j >> 1);
            half = j & 1;
            grp = (wave >> 1) & 1;  // waves 0-3: 32-row position wave & 1, k group
            wq = wave & 1;
        }
    } else {
        logical = xcd_remap(blockIdx.x, gridDim.x);
    }
    const bool active = !TAIL || half < 0 || wave < 4;  // wave-uniform
    int split = 0, tile_id = logical;
    if (SPLIT) split_of(sp, logical, tiles_mn * g.batch, &split, &tile_id);
    const int bz = tile_id / tiles_mn;
    const int t = tile_id - bz * tiles_mn;
    const int m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
    const int M = g.M, K = g.K;
    const int nk_total = (K + kBK - 1) / kBK;
    const int kt0 = SPLIT ? split * sp.ktiles_per_split : 0;
    const int kt1 = SPLIT ? min(nk_total, kt0 + sp.ktiles_per_split) : nk_total;
    const int nk = kt1 - kt0;
    const uint64_t Ab = uniform_ptr(g.A + (int64_t)bz * g.sA), Bb = uniform_ptr(g.B + (int64_t)bz * g.sB);
    const int lda = (int)g.lda, ldb = (int)g.ldb;

    // this lane's chunk of each copy: tile row and clamped column
    int ar[IA], ac[IA], br[IB], bc[IB];
#pragma unroll
    for (int e = 0; e < IA; e++) {
        const int c = (wave * IA + e) * 64 + lane;
        ar[e] = c / (BM / 4);
        ac[e] = min(m0 + (c % (BM / 4)) * 4, M - 4);
    }
#pragma unroll
    for (int e = 0; e < IB; e++) {
        const int c = (wave * IB + e) * 64 + lane;
        br[e] = c / (BN / 4);
        bc[e] = min(n0 + (c % (BN / 4)) * 4, g.n_vec - 4);
    }
    // byte offsets (dispatch keeps them below 2^32); rows past K are clamped
    // to K - 1 on the tile that reaches the end of K
    auto issue = [&](int s, int kt) {
        const int k0 = kt * kBK;
        const bool full = k0 + kBK <= K;
#pragma unroll
        for (int e = 0; e < IA; e++) {
            const int row = full ? k0 + ar[e] : min(k0 + ar[e], K - 1);
            dma16s(Ab, (uint32_t)(row * lda + ac[e]) * 4u, lds_off(As + s * SA + (wave * IA + e) * 256));
        }
#pragma unroll
        for (int e = 0; e < IB; e++) {
            const int row = full ? k0 + br[e] : min(k0 + br[e], K - 1);
            dma16s(Bb, (uint32_t)(row * ldb + bc[e]) * 4u, lds_off(Bs + s * SB + (wave * IB + e) * 256));
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    const int wm0 = (wq % WGM) * WM, wn0 = half >= 0 ? half * 32 : (wq / WGM) * WN;
    const int l32 = lane & 31;
    // this half-wave's k rows of a tile: kr .. kr + 2*KQ... (lanes 32-63 from row 16)
    const int kr = (lane >> 5) * KH + KQ * grp;

    // one tile: rows kr + q, q < KQ, as MFMA k-slot (lane >> 5) of step q
    auto compute = [&](int s) {
        const float *as = As + s * SA + kr * BM + wm0 + l32;
        const float *bs = Bs + s * SB + kr * BN + wn0 + l32;
        float fa[KQ][TM], fb[KQ][TN];
#pragma unroll
        for (int q = 0; q < KQ; q++) {
#pragma unroll
            for (int i = 0; i < TM; i++) fa[q][i] = as[q * BM + i * 32];
#pragma unroll
            for (int j = 0; j < TN; j++) fb[q][j] = bs[q * BN + j * 32];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < KQ; q++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q][i], fb[q][j], acc[i][j], 0, 0, 0);
    };

    // The rows' bias (per-row bias, direct store) is loaded before the k loop:
    // the first tile's wait covers it, and the epilogue does not start with a
    // memory round trip.  Group g of KG = 2 stores registers 8g .. 8g + 7.
    constexpr int ERN = KG == 2 ? 8 : 16;
    const int erb = KG == 2 ? 8 * grp : 0;
    RowBias<TM, ERN> bv;
    const bool pre_bias = !SPLIT && g.bias && !g.bias_n;
    if (pre_bias) load_row_bias(bv, g, m0 + wm0, erb, lane);

    if (nk > 0) {
        const int klast = kt1 - 1;
        const int ktail = K - (nk_total - 1) * kBK;  // valid rows of the global last tile
#pragma unroll
        for (int u = 0; u < NS - 1; u++) issue(u, min(kt0 + u, klast));
        for (int i = 0; i < nk; i++) {
            const int kt = kt0 + i, u = i % NS;
            // this wave's copies of tile kt have landed (NS - 2 younger tiles
            // may stay in flight) ...
            wait_vmcnt<(NS - 2) * (IA + IB)>();
            __syncthreads();  // ... and everyone's; tile kt-1 is consumed
            if (kt == nk_total - 1 && ktail < kBK) {
                for (int x = tid; x < (kBK - ktail) * BM; x += NT) As[u * SA + ktail * BM + x] = 0.0f;
                __syncthreads();
            }
            // into tile kt-1's stage.  With two stages the wait above is
            // vmcnt(0), so the copy past the last tile is simply not issued
            // (the block would otherwise wait for it before its epilogue);
            // deeper pipelines keep a fixed copy count per trip for their
            // vmcnt accounting and repeat the last tile instead.
            if (NS > 2 || i + 1 < nk) issue((i + NS - 1) % NS, min(kt + NS - 1, klast));
            if (active) compute(u);
        }
        wait_vmcnt<0>();  // no copy may still target this block's LDS when it exits
    }
    if constexpr (KG == 2) {
        // The groups' partial tiles are summed through the (now idle) stages
        // and each group finishes half of the rows: group 0 registers 0-7,
        // group 1 registers 8-15 (the same sums as one group adding the
        // other's whole tile; the epilogue's stores split across 8 waves).
        constexpr int HALF = TM * TN * 8 * 64;  // floats one wave hands over
        static_assert(2 * 4 * HALF <= NS * (SA + SB), "reduction space");
        __syncthreads();  // every wave's last compute() has read its operands
        float *give = smem + (grp * 4 + wq) * HALF + lane;
        const float *take = smem + ((1 - grp) * 4 + wq) * HALF + lane;
        if (!active) {
            __syncthreads();  // the working waves' exchange
            return;
        }
        if (grp == 0) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 8; r++) give[((i * TN + j) * 8 + r) * 64] = acc[i][j][8 + r];
        } else {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 8; r++) give[((i * TN + j) * 8 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (grp == 0) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 8; r++) acc[i][j][r] += take[((i * TN + j) * 8 + r) * 64];
            if (pre_bias) {
                gemm_epilogue<TM, TN, SPLIT, 0, 8, true>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane, &bv);
            } else {
                gemm_epilogue<TM, TN, SPLIT, 0, 8>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane);
            }
        } else {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 8; r++) acc[i][j][8 + r] += take[((i * TN + j) * 8 + r) * 64];
            if (pre_bias) {
                gemm_epilogue<TM, TN, SPLIT, 8, 8, true>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane, &bv);
            } else {
                gemm_epilogue<TM, TN, SPLIT, 8, 8>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane);
            }
        }
        return;
    } else {
        if (pre_bias)
            gemm_epilogue<TM, TN, SPLIT, 0, 16, true>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane, &bv);
        else
            gemm_epilogue<TM, TN, SPLIT>(acc, g, sp, split, bz, m0 + wm0, n0 + wn0, lane);
    }
}

// ---------------------------------------------------------------------------
// Implicit-im2col conv with an LDS-staged input patch, for convs with at most
// 32 output channels (the stem): the gather of the generic loader costs index
// arithmetic and a global load per element, here each input element is loaded
// once per block with coalesced rows.  A block owns the 32 output channels of
// one 128-pixel segment of an output row (4 waves x 32 pixels).  Per chunk of
// CC input channels it stages the KS input rows the segment reads (zero outside
// the image: the conv's padding) and the chunk's weights, then runs the MFMAs
// from LDS with k = icl * KS*KS + tap inside the chunk.  Staging issues all of
// a thread's loads before its LDS stores (one memory latency per chunk).  The
// epilogue is bias + act, stored only inside the row.
constexpr int kPatchFloats = 10240, kPatchAFloats = 8192;  // LDS floats per block

template <int KS, int S>
__global__ __launch_bounds__(kThreads) void k_conv_patch(GemmArgs g, int CC, int nseg) {
    constexpr int TW = 128, PW = (TW - 1) * S + KS, TAPS = KS * KS;
    constexpr int JP = kPatchFloats / kThreads, JA = kPatchAFloats / kThreads;
    __shared__ float patch[kPatchFloats];
    __shared__ float As[kPatchAFloats];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int oy = b / nseg, ox0 = (b - oy * nseg) * TW;
    const int M = g.M, IC = g.IC, IH = g.IH, IW = g.IW, OW = g.OW, lda = (int)g.lda;
    const int KC = TAPS * CC, KCp = (KC + 1) & ~1;
    const int iy0 = oy * S - g.P, ix0 = ox0 * S - g.P;
    const float *__restrict__ X = g.B;
    const float *__restrict__ A = g.A;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const int nb = wave * 32 + l32;  // this lane's output column within the segment
    const float *pb = patch + nb * S;

    for (int ic0 = 0; ic0 < IC; ic0 += CC) {
        const int cc = min(CC, IC - ic0);
        const int np = cc * KS * PW, na = KCp * 32;
        float vp[JP], va[JA];
        // Every load is unconditional, at an address clamped into the same
        // row / matrix (one basic block, so the loads stay in flight together;
        // clamping to nearby addresses keeps masked lanes off any shared
        // line), and the mask is applied to the value.
#pragma unroll
        for (int j = 0; j < JP; j++) {
            const int i = min(tid + j * kThreads, np - 1);
            const int row = i / PW, c = i - row * PW;  // row = icl * KS + r
            const int icl = row / KS, r = row - icl * KS;
            const int iy = iy0 + r, ix = ix0 + c;
            const bool in = tid + j * kThreads < np && iy >= 0 && iy < IH && ix >= 0 && ix < IW;
            const float v = X[(uint32_t)((ic0 + icl) * IH * IW + min(max(iy, 0), IH - 1) * IW + min(max(ix, 0), IW - 1))];
            vp[j] = in ? v : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < JA; j++) {
            const int i = tid + j * kThreads;
            const int k = min(i >> 5, KC - 1), m = i & 31;
            const int icl = k / TAPS, tap = k - icl * TAPS;
            const bool in = i < na && (i >> 5) < KC && m < M && icl < cc;
            const float v = A[(uint32_t)((tap * IC + ic0 + min(icl, cc - 1)) * lda + min(m, M - 1))];
            va[j] = in ? v : 0.0f;
        }
        __syncthreads();  // the previous chunk is consumed
#pragma unroll
        for (int j = 0; j < JP; j++) {
            if (tid + j * kThreads < np) patch[tid + j * kThreads] = vp[j];
        }
#pragma unroll
        for (int j = 0; j < JA; j++) {
            if (tid + j * kThreads < na) As[tid + j * kThreads] = va[j];
        }
        __syncthreads();
        // this lane's k = 2*st + hi, stepped by 2 (TAPS is a constant); the
        // pad row k = KC of an odd KC has zero weights and reads offset 0
        int kk = hi, icl = 0, tap = hi;
#pragma unroll 4
        for (int st = 0; st < KCp / 2; st++) {
            const int kh = tap / KS, kw = tap - kh * KS;
            const int off = kk < KC ? (icl * KS + kh) * PW + kw : 0;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[kk * 32 + l32], pb[off], acc, 0, 0, 0);
            kk += 2;
            tap += 2;
            if (tap >= TAPS) {  // TAPS >= 4: at most one carry
                tap -= TAPS;
                ++icl;
            }
        }
    }

    const int ox = ox0 + nb;
    if (ox < OW) {
        float *__restrict__ C = g.C;
        const int64_t pix = (int64_t)oy * OW + ox;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = 8 * (r >> 2) + 4 * hi + (r & 3);
            if (m < M) C[(int64_t)m * g.ldc + pix] = act_f(acc[r] + (g.bias ? g.bias[m] : 0.0f), g.act);
        }
    }
}

// Patch kernel plan: channels per chunk so that the staged rows and weights fit
// (0 = not applicable: more than 32 output channels, or another kernel shape).
// Opt-in (PPDL_CONV_PATCH=1): at ~306 VGPRs and 72 KB of LDS it holds one wave
// per SIMD and measured 2.5-3x slower on the 800x800 stem convolutions than
// the generic implicit-im2col loader, which keeps several waves per SIMD.
int patch_cc(const GemmArgs &g) {
    const char *e = getenv("PPDL_CONV_PATCH");
    if (!(e && e[0] == '1') || g.M > 32 || g.a_rowmajor || g.add || g.c_trans) return 0;
    const int KS = g.KW;
    if (!((KS == 3 && g.S == 2) || (KS == 2 && g.S == 1))) return 0;
    const int PW = 127 * g.S + KS;
    int cc = std::min(g.IC, kPatchFloats / (KS * PW));
    cc = std::min(cc, (kPatchAFloats / 32 - 1) / (KS * KS));  // (KC + 1) rows of 32 weights
    return cc >= 1 ? cc : 0;
}

hipError_t launch_patch(const GemmArgs &g, int cc, hipStream_t s) {
    const int OH = g.N / g.OW, nseg = (g.OW + 127) / 128;
    const int64_t blocks = (int64_t)OH * nseg;
    // the kernel addresses the input and the weights with 32-bit offsets
    if (blocks <= 0 || blocks > 0x7fffffff || (int64_t)g.IC * g.IH * g.IW > 0x7fffffff ||
        (int64_t)g.KW * g.KW * g.IC * g.lda > 0x7fffffff)
        return hipErrorInvalidValue;
    if (g.KW == 3)
        hipLaunchKernelGGL((k_conv_patch<3, 2>), dim3((unsigned)blocks), dim3(kThreads), 0, s, g, cc, nseg);
    else
        hipLaunchKernelGGL((k_conv_patch<2, 1>), dim3((unsigned)blocks), dim3(kThreads), 0, s, g, cc, nseg);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Implicit-im2col conv for at most 32 output channels, operands fetched from
// global memory straight into MFMA operand registers: no LDS staging and no
// barrier in the k loop.  A wave owns the (padded) 32 output channels of 32
// consecutive output pixels; lane l supplies pixel (l & 31) and k slot
// (l >> 5) of every 32x32x2 step.  The k range is walked tap by tap, two
// input channels per step: step s of tap t contracts channels 2s and 2s + 1
// of that tap (k = t*IC + 2s + slot, the .wr row order), so a lane tests its
// pixel's bounds and forms its base address once per tap.  With odd IC the
// last step of a tap has a zero second slot in A and B.  A lane issues the
// loads of kFragU steps before their MFMAs (unconditional, at clamped
// addresses; the masks are applied to the values).  WV waves of a block take
// consecutive parts of the step range for the same 32 pixels and add their
// tiles through LDS in wave order, so the sum order is fixed.
constexpr int kFragU = 16;

template <int WV>
__global__ __launch_bounds__(64 * WV) void k_conv_frag(GemmArgs g) {
    __shared__ float red[WV > 1 ? (WV - 1) * 16 * 64 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, slot = lane >> 5;
    const int grp = xcd_remap(blockIdx.x, gridDim.x);
    const int M = g.M, N = g.N, IC = g.IC, IH = g.IH, IW = g.IW, KW = g.KW;
    const int n = grp * 32 + l32;
    const bool n_ok = n < N;
    const int nc = n_ok ? n : N - 1;
    const int oy = nc / g.OW, ox = nc - oy * g.OW;
    const int iy0 = oy * g.S - g.P, ix0 = ox * g.S - g.P;
    const int ntap = KW * KW, spt = (IC + 1) >> 1;  // taps, steps per tap
    const int nsteps = ntap * spt;
    const int per = (nsteps + WV - 1) / WV;
    const int j0 = min(nsteps, wave * per), j1 = min(nsteps, j0 + per);
    const uint32_t plane = (uint32_t)IH * (uint32_t)IW;
    const float *__restrict__ X = g.B;
    const float *__restrict__ Wt = g.A;
    const uint32_t lda = (uint32_t)g.lda;
    const bool m_ok = l32 < M;
    const uint32_t mc = (uint32_t)min(l32, M - 1);

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;

    // state of the next step: its tap, its step within the tap, and this
    // lane's bounds test and (clamped) input offset for that tap
    int tap = j0 / spt, st = j0 - tap * spt;
    bool in_tap = false;
    uint32_t xb = 0;
    auto enter_tap = [&]() {
        const int t = min(tap, ntap - 1);
        const int kh = t / KW, kw = t - kh * KW;
        const int iy = iy0 + kh, ix = ix0 + kw;
        in_tap = n_ok && tap < ntap && iy >= 0 && iy < IH && ix >= 0 && ix < IW;
        xb = (uint32_t)(min(max(iy, 0), IH - 1) * IW + min(max(ix, 0), IW - 1));
    };
    enter_tap();
    for (int j = j0; j < j1; j += kFragU) {
        float av[kFragU], bv[kFragU];
        bool oka[kFragU], okb[kFragU];
#pragma unroll
        for (int u = 0; u < kFragU; u++) {
            const bool live = j + u < j1;  // wave-uniform
            const int ic = 2 * st + slot;
            const uint32_t icc = (uint32_t)min(ic, IC - 1);
            const uint32_t tc = (uint32_t)min(tap, ntap - 1);
            bv[u] = X[icc * plane + xb];
            av[u] = Wt[(tc * (uint32_t)IC + icc) * lda + mc];
            oka[u] = live && ic < IC && m_ok;
            okb[u] = live && ic < IC && in_tap;
            if (live && ++st == spt) {  // wave-uniform
                st = 0;
                ++tap;
                enter_tap();
            }
        }
#pragma unroll
        for (int u = 0; u < kFragU; u++)
            if (j + u < j1)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(oka[u] ? av[u] : 0.0f, okb[u] ? bv[u] : 0.0f, acc, 0, 0, 0);
    }

    if constexpr (WV > 1) {
        if (wave > 0)
#pragma unroll
            for (int r = 0; r < 16; r++) red[((wave - 1) * 16 + r) * 64 + lane] = acc[r];
        __syncthreads();
        if (wave > 0) return;
        for (int w = 1; w < WV; w++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] += red[((w - 1) * 16 + r) * 64 + lane];
    }
    if (!n_ok) return;
    float *__restrict__ C = g.C;
    const uint32_t ldc = (uint32_t)g.ldc;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = 8 * (r >> 2) + 4 * slot + (r & 3);
        if (m < M) C[(uint32_t)m * ldc + (uint32_t)n] = act_f(acc[r] + (g.bias ? g.bias[m] : 0.0f), g.act);
    }
}

// ---------------------------------------------------------------------------
// k2 s1 p0 convs with 16 or 32 input and at most 32 output channels, OW and
// IW multiples of 4 (the stem's 2x2 convs at 400x400, bottom / right padding
// by clamping), on v_mfma_f32_16x16x4f32.  A lane owns a quad of 4
// consecutive output pixels of one row (lane l: quad l % 16 of the wave's 16)
// and channel slot l / 16 (4 input channels per MFMA step).  Per input row
// (kh) and channel quad, one float4 of the row plus the next column give the
// 5 input values both column taps of the 4 pixels read, so two input loads
// and two weight loads per 16-channel tile feed 8 MFMAs (4 accumulators per
// tile, one per pixel of the quad); all of a row's loads are issued before
// its MFMAs.  Register r of an accumulator holds output channel
// 16 t + 4 (l / 16) + r of quad l % 16, so the 4 accumulators give a float4
// of 4 consecutive pixels per register.  The fragment kernel (32-row tiles,
// one value per operand per MFMA, half-empty tiles at 16 output channels)
// took 30.7 / 21.7 us at 32 -> 16 / 16 -> 32 @400x400.
typedef float f32x4_k2q __attribute__((ext_vector_type(4)));

template <int IC, int MT>
__global__ __launch_bounds__(256) void k_conv_k2q(GemmArgs g) {
    constexpr int NQC = IC / 4;  // channel quads
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int OW = g.OW, IW = g.IW, IH = g.IH, M = g.M;
    const int QW = OW >> 2, NQ = g.N >> 2;
    const int qd = (xcd_remap(blockIdx.x, gridDim.x) * 4 + wave) * 16 + c16;
    const int qc = min(qd, NQ - 1);
    const int oy = qc / QW, ox0 = 4 * (qc - oy * QW);
    const uint32_t plane = (uint32_t)IH * (uint32_t)IW, lda = (uint32_t)g.lda;
    uint32_t mc[MT];
    bool m_ok[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) mc[t] = (uint32_t)min(16 * t + c16, M - 1), m_ok[t] = 16 * t + c16 < M;
    const bool e_in = ox0 + 4 < IW;
    const uint32_t ecol = (uint32_t)min(ox0 + 4, IW - 1) - (uint32_t)ox0;
    const float *__restrict__ X = g.B;
    const float *__restrict__ Wt = g.A;
    f32x4_k2q acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[t][q] = f32x4_k2q{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
        const int iy = oy + kh;
        const bool rin = iy < IH;
        const uint32_t rowo = (uint32_t)min(iy, IH - 1) * (uint32_t)IW + (uint32_t)ox0;
        float4 v[NQC];
        float e[NQC], a0[MT][NQC], a1[MT][NQC];
#pragma unroll
        for (int p = 0; p < NQC; p++) {
            const uint32_t ic = (uint32_t)(4 * p + g4);
            const float *xr = X + ic * plane + rowo;
            v[p] = *reinterpret_cast<const float4 *>(xr);
            e[p] = xr[ecol];
#pragma unroll
            for (int t = 0; t < MT; t++) {
                a0[t][p] = Wt[((uint32_t)(2 * kh) * (uint32_t)IC + ic) * lda + mc[t]];
                a1[t][p] = Wt[((uint32_t)(2 * kh + 1) * (uint32_t)IC + ic) * lda + mc[t]];
            }
        }
#pragma unroll
        for (int p = 0; p < NQC; p++) {
            const float x[5] = {rin ? v[p].x : 0.0f, rin ? v[p].y : 0.0f, rin ? v[p].z : 0.0f, rin ? v[p].w : 0.0f,
                                (rin && e_in) ? e[p] : 0.0f};
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const float w0 = m_ok[t] ? a0[t][p] : 0.0f, w1 = m_ok[t] ? a1[t][p] : 0.0f;
#pragma unroll
                for (int q = 0; q < 4; q++)
                    acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(w0, x[q], acc[t][q], 0, 0, 0);
#pragma unroll
                for (int q = 0; q < 4; q++)
                    acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(w1, x[q + 1], acc[t][q], 0, 0, 0);
            }
        }
    }
    if (qd >= NQ) return;
    float *__restrict__ C = g.C;
    const uint32_t ldc = (uint32_t)g.ldc, px = (uint32_t)oy * (uint32_t)OW + (uint32_t)ox0;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * t + 4 * g4 + r;
            if (m < M) {
                const float b = g.bias ? g.bias[m] : 0.0f;
                const float4 o = make_float4(act_f(acc[t][0][r] + b, g.act), act_f(acc[t][1][r] + b, g.act),
                                             act_f(acc[t][2][r] + b, g.act), act_f(acc[t][3][r] + b, g.act));
                *reinterpret_cast<float4 *>(C + (uint32_t)m * ldc + px) = o;
            }
        }
}

// k3 s2 p1 convs with 64 input and at most 32 output channels (the stem's
// 64 -> 32 conv at 400 -> 200), the same quad scheme: the 4 output pixels of
// a lane read input columns 2 ox0 - 1 .. 2 ox0 + 7 of each of the 3 rows, one
// scalar and two float4 loads, which feed all 3 column taps (tap kw of pixel
// q is element 2 q + kw).  K = 576 is long for one wave, so the block's 4
// waves take a quarter of the input channels each for the same 16 quads and
// add their tiles through LDS in wave order.
template <int IC, int MT>
__global__ __launch_bounds__(256) void k_conv_k3s2q(GemmArgs g) {
    constexpr int NQC = IC / 16;  // channel quads per wave
    __shared__ float red[3][MT * 16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int OW = g.OW, IW = g.IW, IH = g.IH, M = g.M;
    const int QW = OW >> 2, NQ = g.N >> 2;
    const int qd = xcd_remap(blockIdx.x, gridDim.x) * 16 + c16;
    const int qc = min(qd, NQ - 1);
    const int oy = qc / QW, ox0 = 4 * (qc - oy * QW);
    const uint32_t plane = (uint32_t)IH * (uint32_t)IW, lda = (uint32_t)g.lda;
    uint32_t mc[MT];
    bool m_ok[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) mc[t] = (uint32_t)min(16 * t + c16, M - 1), m_ok[t] = 16 * t + c16 < M;
    const bool l_in = ox0 > 0;  // column 2 ox0 - 1 inside the image
    const uint32_t c1 = (uint32_t)(2 * ox0);  // first float4 column
    const float *__restrict__ X = g.B;
    const float *__restrict__ Wt = g.A;
    f32x4_k2q acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[t][q] = f32x4_k2q{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kh = 0; kh < 3; kh++) {
        const int iy = 2 * oy - 1 + kh;
        const bool rin = iy >= 0 && iy < IH;
        const uint32_t rowo = (uint32_t)min(max(iy, 0), IH - 1) * (uint32_t)IW;
        float4 v0[NQC], v1[NQC];
        float xl[NQC], a[MT][3][NQC];
#pragma unroll
        for (int p = 0; p < NQC; p++) {
            const uint32_t ic = (uint32_t)(4 * (wave * NQC + p) + g4);
            const float *xr = X + ic * plane + rowo;
            xl[p] = xr[l_in ? c1 - 1 : c1];
            v0[p] = *reinterpret_cast<const float4 *>(xr + c1);
            v1[p] = *reinterpret_cast<const float4 *>(xr + c1 + 4);
#pragma unroll
            for (int kw = 0; kw < 3; kw++)
#pragma unroll
                for (int t = 0; t < MT; t++) a[t][kw][p] = Wt[((uint32_t)(kh * 3 + kw) * (uint32_t)IC + ic) * lda + mc[t]];
        }
#pragma unroll
        for (int p = 0; p < NQC; p++) {
            const float x[9] = {(rin && l_in) ? xl[p] : 0.0f, rin ? v0[p].x : 0.0f, rin ? v0[p].y : 0.0f,
                                rin ? v0[p].z : 0.0f,         rin ? v0[p].w : 0.0f, rin ? v1[p].x : 0.0f,
                                rin ? v1[p].y : 0.0f,         rin ? v1[p].z : 0.0f, rin ? v1[p].w : 0.0f};
#pragma unroll
            for (int kw = 0; kw < 3; kw++)
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const float w = m_ok[t] ? a[t][kw][p] : 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(w, x[2 * q + kw], acc[t][q], 0, 0, 0);
                }
        }
    }
    // waves 1-3 hand their tiles to wave 0 (register t * 16 + q * 4 + r)
    if (wave > 0)
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 4; r++) red[wave - 1][t * 16 + q * 4 + r][lane] = acc[t][q][r];
    __syncthreads();
    if (wave > 0 || qd >= NQ) return;
#pragma unroll
    for (int w = 0; w < 3; w++)
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[t][q][r] += red[w][t * 16 + q * 4 + r][lane];
    float *__restrict__ C = g.C;
    const uint32_t ldc = (uint32_t)g.ldc, px = (uint32_t)oy * (uint32_t)OW + (uint32_t)ox0;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * t + 4 * g4 + r;
            if (m < M) {
                const float b = g.bias ? g.bias[m] : 0.0f;
                const float4 o = make_float4(act_f(acc[t][0][r] + b, g.act), act_f(acc[t][1][r] + b, g.act),
                                             act_f(acc[t][2][r] + b, g.act), act_f(acc[t][3][r] + b, g.act));
                *reinterpret_cast<float4 *>(C + (uint32_t)m * ldc + px) = o;
            }
        }
}

bool k3s2q_ok(const GemmArgs &g) {
    const char *e = getenv("PPDL_CONV_K2Q");
    if (e && e[0] == '0') return false;
    const auto a16 = [](const void *q) { return (((uintptr_t)q) & 15) == 0; };
    return g.KW == 3 && g.S == 2 && g.P == 1 && g.IC == 64 && g.M >= 1 && g.M <= 32 && !g.a_rowmajor &&
           !g.c_trans && g.add_mode == 0 && !g.add && g.batch == 1 && g.OW >= 4 && g.OW % 4 == 0 &&
           g.IW % 4 == 0 && 2 * g.OW <= g.IW && g.N % g.OW == 0 && g.ldc % 4 == 0 && g.ldc >= g.N && a16(g.B) &&
           a16(g.C) && (int64_t)g.IC * g.IH * g.IW < (1LL << 31) && (int64_t)9 * g.IC * g.lda < (1LL << 31) &&
           (int64_t)32 * g.ldc < (1LL << 31);
}

hipError_t launch_k3s2q(const GemmArgs &g, hipStream_t s) {
    const int64_t blocks = (g.N / 4 + 15) / 16;  // 16 quads per block
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (g.M <= 16) hipLaunchKernelGGL((k_conv_k3s2q<64, 1>), dim3((unsigned)blocks), dim3(256), 0, s, g);
    else hipLaunchKernelGGL((k_conv_k3s2q<64, 2>), dim3((unsigned)blocks), dim3(256), 0, s, g);
    return hipGetLastError();
}

// The quad kernel's cases (PPDL_CONV_K2Q=0 turns it off).
bool k2q_ok(const GemmArgs &g) {
    const char *e = getenv("PPDL_CONV_K2Q");
    if (e && e[0] == '0') return false;
    const auto a16 = [](const void *q) { return (((uintptr_t)q) & 15) == 0; };
    return g.KW == 2 && g.S == 1 && g.P == 0 && (g.IC == 16 || g.IC == 32) && g.M >= 1 && g.M <= 32 &&
           !g.a_rowmajor && !g.c_trans && g.add_mode == 0 && !g.add && g.batch == 1 && g.OW >= 4 && g.OW % 4 == 0 &&
           g.IW % 4 == 0 && g.OW <= g.IW && g.N % g.OW == 0 && g.N / g.OW <= g.IH && g.ldc % 4 == 0 && g.ldc >= g.N &&
           a16(g.B) && a16(g.C) && (int64_t)g.IC * g.IH * g.IW < (1LL << 31) &&
           (int64_t)4 * g.IC * g.lda < (1LL << 31) && (int64_t)32 * g.ldc < (1LL << 31);
}

hipError_t launch_k2q(const GemmArgs &g, hipStream_t s) {
    const int64_t quads = g.N / 4, blocks = (quads + 63) / 64;  // 16 quads per wave
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks);
    if (g.M <= 16) {
        if (g.IC == 16) hipLaunchKernelGGL((k_conv_k2q<16, 1>), grid, dim3(256), 0, s, g);
        else hipLaunchKernelGGL((k_conv_k2q<32, 1>), grid, dim3(256), 0, s, g);
    } else {
        if (g.IC == 16) hipLaunchKernelGGL((k_conv_k2q<16, 2>), grid, dim3(256), 0, s, g);
        else hipLaunchKernelGGL((k_conv_k2q<32, 2>), grid, dim3(256), 0, s, g);
    }
    return hipGetLastError();
}

// The fragment kernel serves op 16 with at most 32 output channels (the stem
// convs), plain bias + act into a CHW output.  PPDL_CONV_FRAG=0 turns it off.
bool frag_ok(const GemmArgs &g) {
    static const bool off = [] {
        const char *e = getenv("PPDL_CONV_FRAG");
        return e && e[0] == '0';
    }();
    return !off && g.M >= 1 && g.M <= 32 && !g.a_rowmajor && !g.c_trans && g.add_mode == 0 && !g.add &&
           g.batch == 1 && g.IC >= 1 && g.N >= 1 && (int64_t)g.IC * g.IH * g.IW < (1LL << 31) &&
           ((int64_t)g.KW * g.KW * g.IC * g.lda + 32) < (1LL << 31) && (int64_t)32 * g.ldc + g.N < (1LL << 31);
}

// waves per 32-pixel group: about 32 steps per wave, within ~8 resident
// waves per SIMD over the whole grid
int frag_waves(const GemmArgs &g) {
    const int64_t groups = (g.N + 31) / 32;
    const int64_t nsteps = (int64_t)g.KW * g.KW * ((g.IC + 1) / 2);
    int wv = 1;
    while (wv < 8 && nsteps > 32 * wv && groups * wv * 2 <= 8192) wv *= 2;
    return wv;
}

hipError_t launch_frag(const GemmArgs &g, hipStream_t s) {
    const int64_t groups = (g.N + 31) / 32;
    if (groups > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)groups);
    switch (frag_waves(g)) {
        case 1: hipLaunchKernelGGL(k_conv_frag<1>, grid, dim3(64), 0, s, g); break;
        case 2: hipLaunchKernelGGL(k_conv_frag<2>, grid, dim3(128), 0, s, g); break;
        case 4: hipLaunchKernelGGL(k_conv_frag<4>, grid, dim3(256), 0, s, g); break;
        default: hipLaunchKernelGGL(k_conv_frag<8>, grid, dim3(512), 0, s, g); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Direct VALU conv for k3 s2 convs with at most 4 input and 32 output
// channels (the first stem conv, 3 -> 32 at 800 -> 400).  At 27 products per
// output it is bound by its output writes (20 MB) and by FMA latency, not by
// the MFMA rate.  A block owns 64 consecutive output pixels (lane = pixel, so
// each store is 256 contiguous bytes) and all 32 output channels; each of its
// two waves computes 16 channels as 16 independent FMA chains over the
// pixel's 3 x 3 x IC window, held in registers.  The weights are staged in
// LDS transposed to one padded row per output channel (read as broadcast
// float4s) from a coalesced read of the .wr rows.
__device__ float kZeroWord = 0.0f;  // read-only in practice: global, not constant, so loads stay global_load

template <int IC>
__global__ __launch_bounds__(128) void k_conv_k3s2(GemmArgs g) {
    constexpr int KK = 9 * IC, KP = (KK + 3) & ~3, MG = 16;
    __shared__ __attribute__((aligned(16))) float ws[32 * KP];
    __shared__ float bs[32];
    const int M = g.M, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lda = (uint32_t)g.lda;
    // all of a thread's weight loads issued together: clamped addresses, the
    // padding zeroed by select (a load under a condition is waited for before
    // the next iteration's)
    constexpr int WI = (32 * KP + 127) / 128;
    float wv[WI];
#pragma unroll
    for (int u = 0; u < WI; u++) {
        const int i = min(tid + 128 * u, 32 * KP - 1), k = i >> 5, m = i & 31;
        wv[u] = g.A[(uint32_t)min(k, KK - 1) * lda + (uint32_t)min(m, M - 1)];
    }
#pragma unroll
    for (int u = 0; u < WI; u++) {
        const int i = tid + 128 * u, k = i >> 5, m = i & 31;
        if (i < 32 * KP) ws[m * KP + k] = (m < M && k < KK) ? wv[u] : 0.0f;
    }
    if (tid < 32) bs[tid] = (g.bias && tid < M) ? g.bias[tid] : 0.0f;
    __syncthreads();

    const int n = blockIdx.x * 64 + lane;
    if (n >= g.N) return;
    const int OW = g.OW, IH = g.IH, IW = g.IW;
    const int oy = n / OW, ox = n - oy * OW;
    const int iy0 = 2 * oy - g.P, ix0 = 2 * ox - g.P;
    const uint32_t plane = (uint32_t)IH * (uint32_t)IW;
    const float *__restrict__ X = g.B;
    float v[KP];
#pragma unroll
    for (int kh = 0; kh < 3; kh++)
#pragma unroll
        for (int kw = 0; kw < 3; kw++)
#pragma unroll
            for (int ic = 0; ic < IC; ic++) {
                // an out-of-bounds tap reads a zero word: the choice is made
                // on the address, so every load is issued unconditionally (a
                // select on the loaded value let the compiler branch around
                // each load and wait for it)
                const int iy = iy0 + kh, ix = ix0 + kw;
                const bool ok = iy >= 0 && iy < IH && ix >= 0 && ix < IW;
                v[(kh * 3 + kw) * IC + ic] =
                    *(ok ? X + (uint32_t)ic * plane + (uint32_t)iy * (uint32_t)IW + (uint32_t)ix : &kZeroWord);
            }
#pragma unroll
    for (int k = KK; k < KP; k++) v[k] = 0.0f;

    const int m0 = wave * MG;
    float a[MG];
#pragma unroll
    for (int j = 0; j < MG; j++) a[j] = bs[m0 + j];
    // one k quad of the 16 channels' weights at a time (a fully unrolled
    // loop kept every weight in registers: 256 VGPRs, one wave per SIMD)
#pragma unroll 1
    for (int q = 0; q < KP / 4; q++)
#pragma unroll
        for (int j = 0; j < MG; j++) {
            const float4 w4 = reinterpret_cast<const float4 *>(ws + (m0 + j) * KP)[q];
            a[j] = fmaf(w4.x, v[4 * q], a[j]);
            a[j] = fmaf(w4.y, v[4 * q + 1], a[j]);
            a[j] = fmaf(w4.z, v[4 * q + 2], a[j]);
            a[j] = fmaf(w4.w, v[4 * q + 3], a[j]);
        }
    float *__restrict__ C = g.C;
    const uint32_t ldc = (uint32_t)g.ldc;
#pragma unroll
    for (int j = 0; j < MG; j++)
        if (m0 + j < M) C[(uint32_t)(m0 + j) * ldc + (uint32_t)n] = act_f(a[j], g.act);
}

// The direct kernel serves op 16 for k3 s2 convs with IC <= 4 and OC <= 32
// (plain bias + act into a CHW output).  PPDL_CONV_DIRECT=0 turns it off.
bool direct_ok(const GemmArgs &g) {
    const char *e = getenv("PPDL_CONV_DIRECT");  // read per call: tests switch it
    const bool off = e && e[0] == '0';
    return !off && g.KW == 3 && g.S == 2 && g.IC >= 1 && g.IC <= 4 && g.M >= 1 && g.M <= 32 && !g.a_rowmajor &&
           !g.c_trans && g.add_mode == 0 && !g.add && g.batch == 1 && g.N >= 1 && g.OW >= 1 && g.N % g.OW == 0 &&
           (int64_t)g.IC * g.IH * g.IW < (1LL << 31) && (int64_t)9 * g.IC * g.lda + 32 < (1LL << 31) &&
           (int64_t)32 * g.ldc + g.N < (1LL << 31);
}

hipError_t launch_direct(const GemmArgs &g, hipStream_t s) {
    const int64_t blocks = ((int64_t)g.N + 63) / 64;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks);
    switch (g.IC) {
        case 1: hipLaunchKernelGGL(k_conv_k3s2<1>, grid, dim3(128), 0, s, g); break;
        case 2: hipLaunchKernelGGL(k_conv_k3s2<2>, grid, dim3(128), 0, s, g); break;
        case 3: hipLaunchKernelGGL(k_conv_k3s2<3>, grid, dim3(128), 0, s, g); break;
        default: hipLaunchKernelGGL(k_conv_k3s2<4>, grid, dim3(128), 0, s, g); break;
    }
    return hipGetLastError();
}

// Split-K fix-up: the GEMM epilogue applied to sum_{s=0..S-1} P[s], s
// ascending.  Partials are [s][batch][M][N]; VEC = 4 needs a plain C with
// ldc == N (four consecutive n share m).
template <int VEC>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float *__restrict__ P, int S, int64_t total,
                                                       GemmArgs g) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
    if (i >= total) return;
    const int64_t MN = (int64_t)g.M * g.N;
    const int bz = (int)(i / MN);
    const int64_t rem = i - (int64_t)bz * MN;
    const int m = (int)(rem / g.N), n = (int)(rem - (int64_t)m * g.N);
    float v[VEC];
#pragma unroll
    for (int u = 0; u < VEC; u++) v[u] = P[i + u];
    for (int s = 1; s < S; s++)
#pragma unroll
        for (int u = 0; u < VEC; u++) v[u] += P[s * total + i + u];
    float *C = g.C + (int64_t)bz * g.sC;
    const float *Ad = g.add ? g.add + (int64_t)bz * g.sC : nullptr;
#pragma unroll
    for (int u = 0; u < VEC; u++) {
        const int nn = n + u;
        const int64_t idx = g.c_trans ? (int64_t)nn * g.ldc + m : (int64_t)m * g.ldc + nn;
        float x = v[u];
        if (g.bias) x += g.bias[g.bias_n ? nn : m];
        if (g.add_mode == 1) x += Ad[idx];
        x = act_f(x, g.act);
        if (g.add_mode == 2) x += Ad[idx];
        else if (g.add_mode == 3) x = refine_box(x, Ad[idx]);
        C[idx] = x;
    }
}

// ---------------------------------------------------------------------------
// Small-GEMM path: for shapes whose 64x64 tiling leaves most of the chip idle
// (the decoder's 300-token linears, the backbone's last stages).  A block owns
// a 32x32 output tile and its WV waves split K: wave w contracts k chunks
// w, w+WV, ... of 32, so the serial MFMA chain per wave is K/WV long (the
// planner picks WV = 4, 8 or 16 from K).  Fragments come straight from global
// memory into registers in MFMA operand order (no LDS staging), with the next
// chunk's loads issued before the current chunk's MFMAs.  The WV partial
// tiles are summed through LDS in fixed wave order (deterministic) and the
// usual epilogue applies.
//
// Operand order per chunk (kb = chunk start): step s = 4c + j (c < 4, j < 4)
// pairs k = kb + 8c + j (lanes 0-31) with k = kb + 8c + 4 + j (lanes 32-63);
// A and B use the same pairing, so the sum covers every k once.  A row-major
// (AMODE 1) is then one float4 per lane per c.  AMODE 2 computes A in the
// loader: A[m][k] = relu(b4[k] + sum_j X[m][j] W4[j][k]) for a 4-column X
// (its row is one float4 per lane, loaded once; W4 and b4 are read as float4
// along k, the same address across a half-wave).
constexpr int kSmallKC = 32;
typedef float f32x4_small __attribute__((ext_vector_type(4)));

template <int AMODE, int WV, bool PRE, bool LN>
__device__ __forceinline__ void gemm_small_body(const GemmArgs &g, int tiles_m, int tiles_mn) {
    constexpr int KC = kSmallKC, NS = KC / 2, NT = WV * 64;
    static_assert(!LN || AMODE == 1, "the row norm prologue reads row-major A");
    __shared__ float red[WV][32][33];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bz = logical / tiles_mn;
    const int t = logical - bz * tiles_mn;
    const int m0 = (t % tiles_m) * 32, n0 = (t / tiles_m) * 32;
    const int M = g.M, N = g.N, K = g.K;
    const int lda = (int)g.lda, ldb = (int)g.ldb;
    const float *__restrict__ A = g.A + (int64_t)bz * g.sA;
    const float *__restrict__ B = g.B + (int64_t)bz * g.sB;
    // prologue add (PRE, row-major A): a_add has A's layout; tiles at or past
    // column a_add_n load it too and select zero (no branch between the
    // loads, which would make the compiler wait for each one)
    const float *__restrict__ A2 = PRE ? g.a_add + (int64_t)bz * g.sA : nullptr;
    const bool pre = PRE && n0 < g.a_add_n;
    const int mc = min(m0 + l32, M - 1), nc = min(n0 + l32, N - 1);
    const int nchunk = (K + KC - 1) / KC;
    const float4 xr = AMODE == 2 ? ld4(A + (uint32_t)(mc * lda)) : float4{0.0f, 0.0f, 0.0f, 0.0f};

    auto load = [&](float (&a)[NS], float (&b)[NS], int ch) {
        const int kb = ch * KC;
#pragma unroll
        for (int c = 0; c < KC / 8; c++) {
            const int k4 = kb + 8 * c + 4 * h;  // this lane's 4 consecutive k
            if (AMODE == 2) {
                const int kk = min(k4, K - 4);
                const float4 w0 = ld4(g.a_w4 + kk), w1 = ld4(g.a_w4 + K + kk);
                const float4 w2 = ld4(g.a_w4 + 2 * K + kk), w3 = ld4(g.a_w4 + 3 * K + kk);
                const float4 bb = ld4(g.a_b4 + kk);
                const bool in = k4 < K;
                const float v[4] = {
                    fmaf(xr.w, w3.x, fmaf(xr.z, w2.x, fmaf(xr.y, w1.x, fmaf(xr.x, w0.x, bb.x)))),
                    fmaf(xr.w, w3.y, fmaf(xr.z, w2.y, fmaf(xr.y, w1.y, fmaf(xr.x, w0.y, bb.y)))),
                    fmaf(xr.w, w3.z, fmaf(xr.z, w2.z, fmaf(xr.y, w1.z, fmaf(xr.x, w0.z, bb.z)))),
                    fmaf(xr.w, w3.w, fmaf(xr.z, w2.w, fmaf(xr.y, w1.w, fmaf(xr.x, w0.w, bb.w))))};
#pragma unroll
                for (int j = 0; j < 4; j++) a[4 * c + j] = in ? fmaxf(v[j], 0.0f) : 0.0f;
            } else if (AMODE == 1) {
                // K % 4 == 0: the 4 k are all inside or all outside
                const uint32_t ai = (uint32_t)(mc * lda + min(k4, K - 4));
                float4 v = ld4(A + ai);
                if (PRE && !LN) {
                    const float4 p = ld4(A2 + ai);
                    v.x += pre ? p.x : 0.0f;
                    v.y += pre ? p.y : 0.0f;
                    v.z += pre ? p.z : 0.0f;
                    v.w += pre ? p.w : 0.0f;
                }
                const bool in = k4 < K;
                a[4 * c + 0] = in ? v.x : 0.0f;
                a[4 * c + 1] = in ? v.y : 0.0f;
                a[4 * c + 2] = in ? v.z : 0.0f;
                a[4 * c + 3] = in ? v.w : 0.0f;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int k = k4 + j;
                    const float v = A[(uint32_t)(min(k, K - 1) * lda + mc)];
                    a[4 * c + j] = k < K ? v : 0.0f;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int k = k4 + j;
                const float v = B[(uint32_t)(min(k, K - 1) * ldb + nc)];
                b[4 * c + j] = k < K ? v : 0.0f;
            }
        }
    };

    // the epilogue's bias and residual operands, fetched now so that their
    // latency overlaps the operand loads (clamped indices: always in range).
    // Only with 8 or 16 waves: with 4, the 8 extra registers cost a wave
    // per SIMD (measured 0.35 us slower per launch on the 1x1 convs).
    const float *__restrict__ bias = g.bias;
    float *__restrict__ C = g.C + (int64_t)bz * g.sC;
    const float *__restrict__ Ad = g.add ? g.add + (int64_t)bz * g.sC : nullptr;
    constexpr int EP = 1024 / NT;
    constexpr bool PF = WV >= 8;
    float eb[EP], ea[EP];
#pragma unroll
    for (int i = 0; i < EP && PF; i++) {
        const int fast = tid & 31, slow = (tid >> 5) + (NT / 32) * i;
        const int mm = g.c_trans ? fast : slow, nn = g.c_trans ? slow : fast;
        const int m = min(m0 + mm, M - 1), n = min(n0 + nn, N - 1);
        const int64_t idx = g.c_trans ? (int64_t)n * g.ldc + m : (int64_t)m * g.ldc + n;
        eb[i] = bias ? bias[g.bias_n ? n : m] : 0.0f;
        ea[i] = g.add_mode && Ad ? Ad[idx] : 0.0f;
    }

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    float a0[NS], b0[NS], a1[NS], b1[NS];
    auto mma = [&](const float (&a)[NS], const float (&b)[NS]) {
#pragma unroll
        for (int st = 0; st < NS; st++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[st], b[st], acc, 0, 0, 0);
    };
    // chunks of this wave: wave, wave + WV, ...; two register stages
    int ch = wave;
    if (!LN && ch < nchunk) load(a0, b0, ch);
    if constexpr (LN) {
        // Row norm of A in the prologue (the decoder's post-residual layer
        // norms, src/ppdoclayout.cpp:550-554): the launch gives every wave
        // exactly one 32-k chunk, so the block holds whole rows.  Mean, then
        // the variance of the centred values (two passes), each as lane
        // sums + the partner half-wave + the waves' partials in wave order;
        // y = (x - mean) / sqrt(var + 1e-5) * gamma + beta.  The blocks of
        // the first column tile store y (ln_out, [M][K]) for later use as a
        // residual; a_add (PRE) is added after the norm.
        __shared__ float lsum[WV][32];
        load(a0, b0, ch);
        float gk[NS], bk[NS], pk[NS];
#pragma unroll
        for (int c = 0; c < KC / 8; c++) {
            const int k4 = ch * KC + 8 * c + 4 * h;
            const float4 gv = ld4(g.ln_g + k4), bv = ld4(g.ln_b + k4);
            const float4 pv = PRE ? ld4(A2 + (uint32_t)(mc * lda + k4)) : float4{0.0f, 0.0f, 0.0f, 0.0f};
            gk[4 * c] = gv.x, gk[4 * c + 1] = gv.y, gk[4 * c + 2] = gv.z, gk[4 * c + 3] = gv.w;
            bk[4 * c] = bv.x, bk[4 * c + 1] = bv.y, bk[4 * c + 2] = bv.z, bk[4 * c + 3] = bv.w;
            pk[4 * c] = pv.x, pk[4 * c + 1] = pv.y, pk[4 * c + 2] = pv.z, pk[4 * c + 3] = pv.w;
        }
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; j++) s += a0[j];
        s += __shfl_xor(s, 32);
        if (h == 0) lsum[wave][l32] = s;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < WV; w++) tot += lsum[w][l32];
        const float mean = tot / (float)K;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; j++) {
            a0[j] -= mean;
            q += a0[j] * a0[j];
        }
        q += __shfl_xor(q, 32);
        __syncthreads();  // every wave has read the sums
        if (h == 0) lsum[wave][l32] = q;
        __syncthreads();
        float qt = 0.0f;
#pragma unroll
        for (int w = 0; w < WV; w++) qt += lsum[w][l32];
        const float scale = 1.0f / sqrtf(qt / (float)K + 1e-5f);
#pragma unroll
        for (int j = 0; j < NS; j++) a0[j] = a0[j] * scale * gk[j] + bk[j];
        if (g.ln_out && n0 == 0 && m0 + l32 < M) {
#pragma unroll
            for (int c = 0; c < KC / 8; c++)
                *reinterpret_cast<float4 *>(g.ln_out + (int64_t)(m0 + l32) * K + ch * KC + 8 * c + 4 * h) =
                    make_float4(a0[4 * c], a0[4 * c + 1], a0[4 * c + 2], a0[4 * c + 3]);
        }
        if (PRE && pre) {
#pragma unroll
            for (int j = 0; j < NS; j++) a0[j] += pk[j];
        }
    }
    while (ch < nchunk) {
        if (ch + WV < nchunk) load(a1, b1, ch + WV);
        __builtin_amdgcn_sched_barrier(0);
        mma(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        ch += WV;
        if (ch >= nchunk) break;
        if (ch + WV < nchunk) load(a0, b0, ch + WV);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        ch += WV;
    }

    // accumulator: lane owns column l32, rows 8(r/4) + 4h + r%4
#pragma unroll
    for (int r = 0; r < 16; r++) red[wave][8 * (r >> 2) + 4 * h + (r & 3)][l32] = acc[r];
    __syncthreads();

    // NT threads x 1024/NT outputs; consecutive threads along the contiguous axis of C
#pragma unroll
    for (int i = 0; i < EP; i++) {
        const int fast = tid & 31, slow = (tid >> 5) + (NT / 32) * i;
        const int mm = g.c_trans ? fast : slow, nn = g.c_trans ? slow : fast;
        const int m = m0 + mm, n = n0 + nn;
        if (m < M && n < N) {
            float v = red[0][mm][nn];
#pragma unroll
            for (int w = 1; w < WV; w++) v += red[w][mm][nn];
            const int64_t idx = g.c_trans ? (int64_t)n * g.ldc + m : (int64_t)m * g.ldc + n;
            const float bv = PF ? eb[i] : (bias ? bias[g.bias_n ? n : m] : 0.0f);
            const float av = PF ? ea[i] : (g.add_mode ? Ad[idx] : 0.0f);
            if (bias) v += bv;
            if (g.add_mode == 1) v += av;
            v = act_f(v, g.act);
            if (g.add_mode == 2) v += av;
            else if (g.add_mode == 3) v = refine_box(v, av);
            C[idx] = v;
        }
    }
}

// The small GEMM in 16 x 32 tiles (two 16x16 blocks, v_mfma_f32_16x16x4f32)
// for the decoder's long-K linears (fc2 K = 1024, the query-position MLP
// K = 512), whose 300 x 256 outputs make only 80 tiles of 32 x 32: twice the
// blocks, half the serial matrix work per CU.  Row-major A (AMODE 1) or the
// computed relu(X W4 + b4) (AMODE 2); K % 32 == 0.  Within a 32-k chunk,
// lane group g = l/16 holds k = kb + 8g .. kb + 8g + 7 of its row (two
// float4 loads) and step j contracts k = kb + j, kb + 8 + j, kb + 16 + j,
// kb + 24 + j (group g supplies the g-th of them); B uses the same pairing.
// The WV waves' partial tiles are summed through LDS in wave order.
template <int AMODE, int WV, bool LN, bool PRE>
__global__ __launch_bounds__(WV * 64) void k_gemm_small16(GemmArgs g, int tiles_m, int tiles_mn) {
    constexpr int KC = kSmallKC, NT = WV * 64;
    static_assert(!(LN || PRE) || AMODE == 1, "norm and prologue add read row-major A");
    __shared__ float red[WV][16][33];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, grp = lane >> 4;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bz = logical / tiles_mn;
    const int t = logical - bz * tiles_mn;
    const int m0 = (t % tiles_m) * 16, n0 = (t / tiles_m) * 32;
    const int M = g.M, N = g.N, K = g.K;
    const int lda = (int)g.lda, ldb = (int)g.ldb;
    const float *__restrict__ A = g.A + (int64_t)bz * g.sA;
    const float *__restrict__ B = g.B + (int64_t)bz * g.sB;
    const int mc = min(m0 + l16, M - 1), nc0 = min(n0 + l16, N - 1), nc1 = min(n0 + 16 + l16, N - 1);
    const int nchunk = K / KC;
    float4 xr = AMODE >= 2 ? ld4(A + (uint32_t)(mc * lda)) : float4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (AMODE == 3) {
        // the previous layer's last box-head linear and the box refinement:
        // d_j = box_b[j] + box_h[row] . box_w[:, j] over box_k = 256, each of
        // the block's 32 threads per row taking 8 k (wave w, group g: k from
        // 8 (4 w + g)), summed over the lane groups then the waves in order
        static_assert(WV == 8, "32 threads x 8 k per row");
        __shared__ float bsum[WV][16][4];
        const int kb = 8 * (4 * wave + grp);
        const float *hr = g.box_h + (uint32_t)(mc * g.box_ldh + kb);
        const float4 h0 = ld4(hr), h1 = ld4(hr + 4);
        const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        float d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 w = ld4(g.box_w + 4 * (kb + j));
            d[0] = fmaf(hv[j], w.x, d[0]);
            d[1] = fmaf(hv[j], w.y, d[1]);
            d[2] = fmaf(hv[j], w.z, d[2]);
            d[3] = fmaf(hv[j], w.w, d[3]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            d[j] += __shfl_xor(d[j], 16);
            d[j] += __shfl_xor(d[j], 32);
        }
        if (grp == 0)
#pragma unroll
            for (int j = 0; j < 4; j++) bsum[wave][l16][j] = d[j];
        __syncthreads();
        float t4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float sacc = 0.0f;
#pragma unroll
            for (int w = 0; w < WV; w++) sacc += bsum[w][l16][j];
            t4[j] = sacc + g.box_b[j];
        }
        xr = make_float4(refine_box(t4[0], xr.x), refine_box(t4[1], xr.y), refine_box(t4[2], xr.z),
                         refine_box(t4[3], xr.w));
        if (n0 == 0 && wave == 0 && grp == 0 && m0 + l16 < M)
            *reinterpret_cast<float4 *>(g.box_out + (uint32_t)(4 * (m0 + l16))) = xr;
    }
    // prologue add (row-major A): a_add has A's layout; whole 32-column
    // tiles at or past a_add_n skip it
    const float *__restrict__ A2 = PRE ? g.a_add + (int64_t)bz * g.sA : nullptr;
    const bool pre = PRE && n0 < g.a_add_n;

    auto load = [&](float (&a)[8], float (&b0)[8], float (&b1)[8], int ch) {
        const int k8 = ch * KC + 8 * grp;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int k4 = k8 + 4 * h;
            if (AMODE >= 2) {
                const float4 w0 = ld4(g.a_w4 + k4), w1 = ld4(g.a_w4 + K + k4);
                const float4 w2 = ld4(g.a_w4 + 2 * K + k4), w3 = ld4(g.a_w4 + 3 * K + k4);
                const float4 bb = ld4(g.a_b4 + k4);
                a[4 * h + 0] = fmaxf(fmaf(xr.w, w3.x, fmaf(xr.z, w2.x, fmaf(xr.y, w1.x, fmaf(xr.x, w0.x, bb.x)))), 0.0f);
                a[4 * h + 1] = fmaxf(fmaf(xr.w, w3.y, fmaf(xr.z, w2.y, fmaf(xr.y, w1.y, fmaf(xr.x, w0.y, bb.y)))), 0.0f);
                a[4 * h + 2] = fmaxf(fmaf(xr.w, w3.z, fmaf(xr.z, w2.z, fmaf(xr.y, w1.z, fmaf(xr.x, w0.z, bb.z)))), 0.0f);
                a[4 * h + 3] = fmaxf(fmaf(xr.w, w3.w, fmaf(xr.z, w2.w, fmaf(xr.y, w1.w, fmaf(xr.x, w0.w, bb.w)))), 0.0f);
            } else {
                float4 v = ld4(A + (uint32_t)(mc * lda + k4));
                if (PRE && !LN) {
                    const float4 p = ld4(A2 + (uint32_t)(mc * lda + k4));
                    v.x += pre ? p.x : 0.0f;
                    v.y += pre ? p.y : 0.0f;
                    v.z += pre ? p.z : 0.0f;
                    v.w += pre ? p.w : 0.0f;
                }
                a[4 * h + 0] = v.x, a[4 * h + 1] = v.y, a[4 * h + 2] = v.z, a[4 * h + 3] = v.w;
            }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            b0[j] = B[(uint32_t)((k8 + j) * ldb + nc0)];
            b1[j] = B[(uint32_t)((k8 + j) * ldb + nc1)];
        }
    };
    f32x4_small acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    auto mma = [&](const float (&a)[8], const float (&b0)[8], const float (&b1)[8]) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b0[j], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b1[j], acc1, 0, 0, 0);
        }
    };
    float a0[8], p0[8], q0[8], a1[8], p1[8], q1[8];
    int ch = wave;
    if (!LN && ch < nchunk) load(a0, p0, q0, ch);
    if constexpr (LN) {
        // the row norm of the small GEMM's prologue, on 16-row tiles: every
        // wave holds one 32-k chunk of the 16 rows (the launch gives
        // nchunk == WV); lane sums, the row's four lane groups (xor 16, 32),
        // then the waves' partials in wave order; two passes
        __shared__ float lsum[WV][16];
        load(a0, p0, q0, ch);
        const int k8 = ch * KC + 8 * grp;
        float gk[8], bk[8], pk[8];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float4 gv = ld4(g.ln_g + k8 + 4 * hh), bv = ld4(g.ln_b + k8 + 4 * hh);
            const float4 pv = PRE ? ld4(A2 + (uint32_t)(mc * lda + k8 + 4 * hh)) : float4{0.0f, 0.0f, 0.0f, 0.0f};
            gk[4 * hh] = gv.x, gk[4 * hh + 1] = gv.y, gk[4 * hh + 2] = gv.z, gk[4 * hh + 3] = gv.w;
            bk[4 * hh] = bv.x, bk[4 * hh + 1] = bv.y, bk[4 * hh + 2] = bv.z, bk[4 * hh + 3] = bv.w;
            pk[4 * hh] = pv.x, pk[4 * hh + 1] = pv.y, pk[4 * hh + 2] = pv.z, pk[4 * hh + 3] = pv.w;
        }
        float sm = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) sm += a0[j];
        sm += __shfl_xor(sm, 16);
        sm += __shfl_xor(sm, 32);
        if (grp == 0) lsum[wave][l16] = sm;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < WV; w++) tot += lsum[w][l16];
        const float mean = tot / (float)K;
        float qq = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            a0[j] -= mean;
            qq += a0[j] * a0[j];
        }
        qq += __shfl_xor(qq, 16);
        qq += __shfl_xor(qq, 32);
        __syncthreads();  // every wave has read the sums
        if (grp == 0) lsum[wave][l16] = qq;
        __syncthreads();
        float qt = 0.0f;
#pragma unroll
        for (int w = 0; w < WV; w++) qt += lsum[w][l16];
        const float scale = 1.0f / sqrtf(qt / (float)K + 1e-5f);
#pragma unroll
        for (int j = 0; j < 8; j++) a0[j] = a0[j] * scale * gk[j] + bk[j];
        if (g.ln_out && n0 == 0 && m0 + l16 < M) {
            float *o = g.ln_out + (int64_t)(m0 + l16) * K + k8;
            *reinterpret_cast<float4 *>(o) = make_float4(a0[0], a0[1], a0[2], a0[3]);
            *reinterpret_cast<float4 *>(o + 4) = make_float4(a0[4], a0[5], a0[6], a0[7]);
        }
        if (PRE && pre) {
#pragma unroll
            for (int j = 0; j < 8; j++) a0[j] += pk[j];
        }
    }
    while (ch < nchunk) {
        if (ch + WV < nchunk) load(a1, p1, q1, ch + WV);
        __builtin_amdgcn_sched_barrier(0);
        mma(a0, p0, q0);
        __builtin_amdgcn_sched_barrier(0);
        ch += WV;
        if (ch >= nchunk) break;
        if (ch + WV < nchunk) load(a0, p0, q0, ch + WV);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, p1, q1);
        __builtin_amdgcn_sched_barrier(0);
        ch += WV;
    }
    // result register r of lane l: row 4*(l/16) + r, column l%16 of its block
#pragma unroll
    for (int r = 0; r < 4; r++) {
        red[wave][4 * grp + r][l16] = acc0[r];
        red[wave][4 * grp + r][16 + l16] = acc1[r];
    }
    __syncthreads();
    float *__restrict__ C = g.C + (int64_t)bz * g.sC;
    const float *__restrict__ Ad = g.add ? g.add + (int64_t)bz * g.sC : nullptr;
    for (int e = tid; e < 16 * 32; e += NT) {
        const int mm = e >> 5, nn = e & 31, m = m0 + mm, n = n0 + nn;
        if (m < M && n < N) {
            float v = red[0][mm][nn];
#pragma unroll
            for (int w = 1; w < WV; w++) v += red[w][mm][nn];
            const int64_t idx = (int64_t)m * g.ldc + n;
            if (g.bias) v += g.bias[g.bias_n ? n : m];
            if (g.add_mode == 1) v += Ad[idx];
            v = act_f(v, g.act);
            if (g.add_mode == 2) v += Ad[idx];
            else if (g.add_mode == 3) v = refine_box(v, Ad[idx]);
            C[idx] = v;
        }
    }
}

// The 16 x 32 small GEMM where the 32 x 32 one would leave fewer than 400
// blocks and K >= 256 (PPDL_SMALL16=0 turns it off, =<k> sets the K bound,
// PPDL_SMALL16_T the block bound, for A/B runs; read per call).  Same-process
// graph A/B: K >= 512 (fc2, qpos.1) 37 us per image faster; K >= 256 (also
// sa.o, ca.op, the box and mask-query heads) 25 us more; K >= 32 7 us slower
// than K >= 256; a bound of 400 instead of 128 blocks (adds sa.qkv, fc1) 3 us;
// 700 (adds AIFI's qkv and fc1, 480 and 640 tiles) 3.4 us once the kernel ran
// 8 waves (with 16 it had been 8 us slower).
bool small16_ok(const GemmArgs &g, int amode) {
    const char *e = getenv("PPDL_SMALL16");
    if (e && e[0] == '0') return false;
    const int64_t t32 = (int64_t)((g.M + 31) / 32) * ((g.N + 31) / 32) * g.batch;
    const auto a16 = [](const void *q) { return (((uintptr_t)q) & 15) == 0; };
    const int64_t kmin = (e && *e && e[0] != '0') ? atoi(e) : 256;
    const char *et = getenv("PPDL_SMALL16_T");
    const int64_t tmax = (et && *et) ? atoi(et) : 700;
    return (amode == 1 || amode == 2) && g.K >= kmin && g.K % kSmallKC == 0 && t32 < tmax && !g.c_trans && !g.bits &&
           (amode == 1 || !g.ln_g) && (!g.ln_g || g.K == 8 * kSmallKC) &&
           (!g.a_add || (a16(g.a_add) && g.a_add_n % 32 == 0)) && g.lda % 4 == 0 && a16(g.A) &&
           (int64_t)g.M * g.lda + g.K < 0x7fffffff && (int64_t)g.K * g.ldb + g.N < 0x7fffffff;
}

hipError_t launch_small16(const GemmArgs &g, int amode, hipStream_t s) {
    const int tiles_m = (g.M + 15) / 16, tiles_n = (g.N + 31) / 32, tmn = tiles_m * tiles_n;
    const int64_t total = (int64_t)tmn * g.batch;
    if (total <= 0 || total > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)total);
    // 8 waves with the computed A (16 would cap each wave at 128 registers:
    // spills); the row norm needs one 32-k chunk per wave
    if (amode == 2 && g.box_h)
        hipLaunchKernelGGL((k_gemm_small16<3, 8, false, false>), grid, dim3(512), 0, s, g, tiles_m, tmn);
    else if (amode == 2) hipLaunchKernelGGL((k_gemm_small16<2, 8, false, false>), grid, dim3(512), 0, s, g, tiles_m, tmn);
    else if (g.ln_g && g.a_add)
        hipLaunchKernelGGL((k_gemm_small16<1, 8, true, true>), grid, dim3(512), 0, s, g, tiles_m, tmn);
    else if (g.ln_g) hipLaunchKernelGGL((k_gemm_small16<1, 8, true, false>), grid, dim3(512), 0, s, g, tiles_m, tmn);
    // 8 waves: at K = 256 one 32-k chunk each (16 left half of them idle:
    // graph -13 us), at K = 1024 four each (-4 us against 16 waves with
    // two); PPDL_SMALL16_WV16=1 keeps 16
    else {
        const char *ew = getenv("PPDL_SMALL16_WV16");
        const bool w8 = !(ew && ew[0] == '1');
        if (g.a_add && w8)
            hipLaunchKernelGGL((k_gemm_small16<1, 8, false, true>), grid, dim3(512), 0, s, g, tiles_m, tmn);
        else if (g.a_add)
            hipLaunchKernelGGL((k_gemm_small16<1, 16, false, true>), grid, dim3(1024), 0, s, g, tiles_m, tmn);
        else if (w8)
            hipLaunchKernelGGL((k_gemm_small16<1, 8, false, false>), grid, dim3(512), 0, s, g, tiles_m, tmn);
        else hipLaunchKernelGGL((k_gemm_small16<1, 16, false, false>), grid, dim3(1024), 0, s, g, tiles_m, tmn);
    }
    return hipGetLastError();
}

template <int AMODE, int WV, bool PRE>
__global__ __launch_bounds__(WV * 64) void k_gemm_small(GemmArgs g, int tiles_m, int tiles_mn) {
    gemm_small_body<AMODE, WV, PRE, false>(g, tiles_m, tiles_mn);
}

// the small GEMM with the row-norm prologue (row-major A, K = 32 * WV)
template <int WV, bool PRE>
__global__ __launch_bounds__(WV * 64) void k_gemm_small_ln(GemmArgs g, int tiles_m, int tiles_mn) {
    gemm_small_body<1, WV, PRE, true>(g, tiles_m, tiles_mn);
}

// Waves of the small-GEMM kernel (PPDL_SMALL_WV pins 4, 8 or 16 for sweeps
// and tests).  Measured on the network's shapes: with 256 or more 32x32
// tiles the grid already fills the chip and 4 waves per tile won (less LDS
// reduction, more blocks resident); below that, splitting K as far as one or
// two 32-k chunks per wave won (the 300-token decoder linears: 5.8 -> 4.8 us
// at K = 256, 12.7 -> 10.9 us at K = 1024).
int small_waves(int K, int64_t tiles) {
    const char *e = getenv("PPDL_SMALL_WV");
    if (e && *e) {
        const int w = atoi(e);
        if (w == 1 || w == 2 || w == 4 || w == 8 || w == 16) return w;
    }
    const int nchunk = (K + kSmallKC - 1) / kSmallKC;
    if (tiles >= 256 || nchunk <= 4) return 4;
    return nchunk <= 8 ? 8 : 16;
}

int64_t small_tiles(const GemmArgs &g) { return (int64_t)((g.M + 31) / 32) * ((g.N + 31) / 32) * g.batch; }

struct TileCfg {
    int bm, bn, wgm;
};
// Block shapes (BM, BN, waves along M); wave tiles 64x64 .. 32x32.
constexpr TileCfg kCfgs[] = {
    {128, 128, 2},  // 0: wave 64x64
    {64, 128, 2},   // 1: wave 32x64
    {128, 64, 2},   // 2: wave 64x32
    {64, 64, 2},    // 3: wave 32x32
    {32, 256, 1},   // 4: wave 32x64
    {32, 128, 1},   // 5: wave 32x32
};
constexpr int kNumCfg = sizeof(kCfgs) / sizeof(kCfgs[0]);
constexpr int kCfgSmall = kNumCfg;  // the small-GEMM kernel (32x32 tiles, K split over waves)
constexpr int kSplitChoices[] = {1, 2, 3, 4, 6, 8, 12, 16};

int64_t tiles_of(int c, int M, int N, int batch) {
    return (int64_t)((M + kCfgs[c].bm - 1) / kCfgs[c].bm) * ((N + kCfgs[c].bn - 1) / kCfgs[c].bn) * batch;
}

// Plan from a sweep of every (block shape, splits) pair on the network's
// GEMM shapes (1x1 convs 64..2048 x 625..40000 x 64..3328, the F(4,3)
// planes, the k2/k3-s2 im2col convs).  64x64 blocks (four resident per CU)
// won or tied nearly everywhere; 32-row blocks when M <= 32.  Splitting K
// paid only when the output had too few tiles to occupy the chip: the best
// S kept about 1000 blocks in flight with at least 6 k tiles per split.
// integer tuning knob from the environment (planner sweeps only)
int64_t env_int(const char *name, int64_t dflt) {
    const char *e = getenv(name);
    return (e && *e) ? strtoll(e, nullptr, 10) : dflt;
}

GemmPlan plan_auto(int M, int N, int K, int batch, bool im2col) {
    // Few output tiles and a small operand footprint: the small-GEMM kernel
    // (32x32 tiles, K split over the block's waves, no split-K pass).  Its
    // L2 traffic grows with the tile count (each operand is re-read once per
    // 32-wide strip of the other), hence the footprint bound.  Bounds from a
    // network sweep (200/40, 400/80, 700/160 tiles/MB): 400/80 was fastest.
    const int64_t t64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64) * batch;
    const int64_t reread = 4 * ((int64_t)M * K * ((N + 31) / 32) + (int64_t)K * N * ((M + 31) / 32)) * batch;
    const int64_t small_t64 = env_int("PPDL_SMALL_T64", 400);  // read per plan: in-process A/B
    const int64_t small_mb = env_int("PPDL_SMALL_MB", 80);
    if (!im2col && t64 < small_t64 && reread <= (small_mb << 20)) return GemmPlan{kCfgSmall, 1};
    GemmPlan p{M <= 32 ? 5 : 3, 1};
    const int nk = (K + kBK - 1) / kBK;
    const int64_t tiles = tiles_of(p.cfg, M, N, batch);
    const int64_t target = env_int("PPDL_SPLIT_BLOCKS", 1000);
    const int64_t min_kt = env_int("PPDL_SPLIT_MIN_KT", 6);
    int64_t want = target / (tiles > 0 ? tiles : 1);
    const int64_t cap = nk / min_kt;
    if (want > cap) want = cap;
    for (int S : kSplitChoices)
        if (S <= want) p.splits = S;
    return p;
}

// PPDL_GEMM_TILE="cfg,splits" pins the plan (tile-shape tuning sweeps only).
int env_override(int *cfg, int *splits) {
    const char *e = getenv("PPDL_GEMM_TILE");
    if (!e || !*e) return 0;
    char *end = nullptr;
    const int oc = (int)strtol(e, &end, 10);
    const int os = (end && *end == ',') ? (int)strtol(end + 1, nullptr, 10) : 1;
    if (oc < 0 || oc > kCfgSmall) return 0;
    *cfg = oc;
    *splits = os < 1 ? 1 : os;
    return 1;
}

// Columns of a dense B row readable as whole float4s: N when N % 4 == 0, N
// rounded up to 4 when the row stride leaves room (padded planes), else 0.
int n_vec_of(const GemmArgs &g) {
    const int n4 = (g.N + 3) & ~3;
    return g.N % 4 == 0 ? g.N : (g.ldb >= n4 ? n4 : 0);
}

// The direct-to-LDS kernel applies to dense k-major operands with 4-aligned
// extents and 16-byte aligned bases (PPDL_GEMM_DMA=0 turns it off).
bool dma_ok(const GemmArgs &g) {
    static const bool off = [] {
        const char *e = getenv("PPDL_GEMM_DMA");
        return e && e[0] == '0';
    }();
    const auto a16 = [](const void *p) { return (((uintptr_t)p) & 15) == 0; };
    // copies address one batch plane with 32-bit byte offsets
    const bool fits = ((int64_t)g.K * g.lda + g.M) * 4 < (1LL << 32) && ((int64_t)g.K * g.ldb + g.N + 4) * 4 < (1LL << 32);
    return !off && !g.a_rowmajor && g.M >= 4 && g.M % 4 == 0 && n_vec_of(g) >= 4 && g.lda % 4 == 0 &&
           g.ldb % 4 == 0 && g.sA % 4 == 0 && g.sB % 4 == 0 && a16(g.A) && a16(g.B) && fits;
}

// Wave groups of the direct-to-LDS kernel: 2 (8 waves per block) where each
// wave still gets a 16-byte copy per operand; PPDL_DMA_KG=1 keeps 4 waves.
// Measured on the network: 3.864 -> 3.859 ms; single 1x1 convs up to 14%
// (K=512 N=10000 M=512: 83 -> 95 TF/s), none slower by more than noise.
int dma_groups() {
    static const int kg = (int)env_int("PPDL_DMA_KG", 2);
    return kg == 1 ? 1 : 2;
}

// CUs per XCD of the current device (blocks go to the 8 XCDs round-robin), 0
// if unknown
int cus_per_xcd() {
    static int cached[16] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 0;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
        cached[dev] = n >= 16 ? n / 8 : -1;
    }
    return cached[dev] > 0 ? cached[dev] : 0;
}

// Grid of the tail-balanced 64x64 launch for T tiles: 8 x the largest
// per-XCD block count, or 0 when no XCD has a remainder of at most half its
// CUs (PPDL_DMA_TAIL=0 turns the mode off; read at every launch, so a test
// can compare both modes in one process).
int64_t tail_grid(int64_t T) {
    const char *e = getenv("PPDL_DMA_TAIL");
    const bool off = e && e[0] == '0';
    const int cus = cus_per_xcd();
    if (off || cus < 2 || T < 8 || T > 0x3fffffff) return 0;
    int64_t most = 0;
    bool any = false;
    for (int x = 0; x < 8; x++) {
        const int64_t cnt = T / 8 + (x < T % 8 ? 1 : 0);
        const int64_t r = cnt % cus, h = (r > 0 && 2 * r <= cus) ? r : 0;
        any = any || h > 0;
        most = std::max(most, cnt + h);
    }
    return any ? 8 * most : 0;
}

// Split launches order their blocks split-major (PPDL_SPLIT_ORDER=tile keeps
// the S splits of a tile adjacent; read at every launch for A/B runs).
int split_major_order() {
    const char *e = getenv("PPDL_SPLIT_ORDER");
    return (e && e[0] == 't') ? 0 : 1;
}

template <int BM, int BN, int WGM, bool SPLIT>
void launch_dma(const GemmArgs &g, const SplitArgs &sp, int64_t total, int tiles_m, int tiles_n, hipStream_t s) {
    // 8 waves need at least one 16-byte copy per operand and wave
    if constexpr (kBK * BM / 4 >= 2 * kThreads && kBK * BN / 4 >= 2 * kThreads) {
        if (dma_groups() == 2) {
            if constexpr (BM == 64 && BN == 64 && WGM == 2 && !SPLIT) {
                if (const int64_t grid = tail_grid(total)) {
                    hipLaunchKernelGGL((k_gemm_dma<64, 64, 2, false, 2, 2, true>), dim3((unsigned)grid),
                                       dim3(2 * kThreads), 0, s, g, sp, tiles_m, tiles_m * tiles_n, cus_per_xcd());
                    return;
                }
            }
            hipLaunchKernelGGL((k_gemm_dma<BM, BN, WGM, SPLIT, 2, 2>), dim3((unsigned)total), dim3(2 * kThreads), 0,
                               s, g, sp, tiles_m, tiles_m * tiles_n, 0);
            return;
        }
    }
    hipLaunchKernelGGL((k_gemm_dma<BM, BN, WGM, SPLIT, 2, 1>), dim3((unsigned)total), dim3(kThreads), 0, s, g, sp,
                       tiles_m, tiles_m * tiles_n, 0);
}

template <int BM, int BN, int WGM, int AMODE, int BMODE>
hipError_t launch(const GemmArgs &g, int S, const GemmWorkspace &ws, hipStream_t s) {
    const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
    const int64_t tiles = (int64_t)tiles_m * tiles_n * g.batch;
    const int64_t total = tiles * S;
    if (total <= 0 || total > 0x7fffffff) return hipErrorInvalidValue;
    // the kernel addresses A and B within one batch plane with 32-bit offsets
    const int64_t a_ext = AMODE == 0 ? (int64_t)g.K * g.lda : (int64_t)g.M * g.lda;
    const int64_t b_ext = BMODE == 0 ? (int64_t)g.K * g.ldb : (int64_t)g.IC * g.IH * g.IW;  // im2col: the image
    if (a_ext + BM > 0x7fffffff || b_ext + BN > 0x7fffffff) return hipErrorInvalidValue;
    SplitArgs sp{1, 0, nullptr, 0};
    if (S > 1) {
        const int nk = (g.K + kBK - 1) / kBK;
        sp.splits = S;
        sp.split_major = split_major_order();
        sp.ktiles_per_split = (nk + S - 1) / S;
        sp.partials = (float *)ws.base;
        if (AMODE == 0 && BMODE == 0 && dma_ok(g))
            launch_dma<BM, BN, WGM, true>(g, sp, total, tiles_m, tiles_n, s);
        else
            hipLaunchKernelGGL((k_gemm<BM, BN, WGM, AMODE, BMODE, true>), dim3((unsigned)total), dim3(kThreads), 0,
                               s, g, sp, tiles_m, tiles_m * tiles_n);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t n = (int64_t)g.M * g.N * g.batch;
        const bool vec = !g.c_trans && g.ldc == g.N && (g.N % 4 == 0) && ((((uintptr_t)g.C) & 15) == 0);
        if (vec)
            hipLaunchKernelGGL(k_splitk_reduce<4>, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s,
                               sp.partials, S, n, g);
        else
            hipLaunchKernelGGL(k_splitk_reduce<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                               sp.partials, S, n, g);
    } else if (AMODE == 0 && BMODE == 0 && dma_ok(g)) {
        launch_dma<BM, BN, WGM, false>(g, sp, total, tiles_m, tiles_n, s);
    } else {
        hipLaunchKernelGGL((k_gemm<BM, BN, WGM, AMODE, BMODE, false>), dim3((unsigned)total), dim3(kThreads), 0,
                           s, g, sp, tiles_m, tiles_m * tiles_n);
    }
    return hipGetLastError();
}

template <int AMODE, bool PRE>
hipError_t launch_small_wv(const GemmArgs &g, int wv, dim3 grid, int tiles_m, int tmn, hipStream_t s) {
    if (wv == 1) hipLaunchKernelGGL((k_gemm_small<AMODE, 1, PRE>), grid, dim3(64), 0, s, g, tiles_m, tmn);
    else if (wv == 2) hipLaunchKernelGGL((k_gemm_small<AMODE, 2, PRE>), grid, dim3(128), 0, s, g, tiles_m, tmn);
    else if (wv == 4) hipLaunchKernelGGL((k_gemm_small<AMODE, 4, PRE>), grid, dim3(256), 0, s, g, tiles_m, tmn);
    else if (wv == 8) hipLaunchKernelGGL((k_gemm_small<AMODE, 8, PRE>), grid, dim3(512), 0, s, g, tiles_m, tmn);
    else hipLaunchKernelGGL((k_gemm_small<AMODE, 16, PRE>), grid, dim3(1024), 0, s, g, tiles_m, tmn);
    return hipGetLastError();
}

template <int AMODE>
hipError_t launch_small(const GemmArgs &g, hipStream_t s) {
    if constexpr (AMODE != 0)
        if (small16_ok(g, AMODE)) return launch_small16(g, AMODE, s);
    const int tiles_m = (g.M + 31) / 32, tiles_n = (g.N + 31) / 32;
    const int64_t total = (int64_t)tiles_m * tiles_n * g.batch;
    const int64_t a_ext = AMODE == 0 ? (int64_t)g.K * g.lda : (int64_t)g.M * g.lda;
    if (total <= 0 || total > 0x7fffffff || a_ext > 0x7fffffff || (int64_t)g.K * g.ldb > 0x7fffffff)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)total);
    const int wv = small_waves(g.K, total), tmn = tiles_m * tiles_n;
    if constexpr (AMODE == 1)
        if (g.a_add) return launch_small_wv<AMODE, true>(g, wv, grid, tiles_m, tmn, s);
    return launch_small_wv<AMODE, false>(g, wv, grid, tiles_m, tmn, s);
}

// Where the 16x16-MFMA tile menu (gemm_lt.hip) replaces the plan: single
// 1x1 convs on maps of at most 4096 pixels that the plan would split along K
// with K <= 1536 (one pass instead of split partials plus a reduction
// launch).  In-graph kernel traces on the network: enc_in1 44 -> 28 us,
// stage-3 agg1 62 -> 46 us, the 1024-channel stage-2 l0 1x1s 22 -> 20 us.
// Where it lost in the graph: the 4-wave small-kernel shapes (8.0 -> 8.7 us;
// faster only in isolated back-to-back replays), the batched F(4,3) planes,
// the 25x25 shapes of the 16-wave small kernel, the unsplit 64x64 GEMMs and
// the long-K (>= 1664) split aggregations.
bool lt_wanted(const GemmArgs &g, const GemmPlan &p) {
    return g.batch == 1 && g.N <= 4096 && p.cfg != kCfgSmall && p.splits > 1 && g.K <= 1536;
}

// the small GEMM with the row-norm prologue: one 32-k chunk per wave
bool ln_ok(const GemmArgs &g) {
    const auto a16 = [](const void *q) { return (((uintptr_t)q) & 15) == 0; };
    const int wv = g.K / kSmallKC;
    return g.a_rowmajor && !g.a_w4 && !g.bits && g.ln_b && g.batch == 1 && g.K % kSmallKC == 0 &&
           (wv == 8 || wv == 16) && g.lda % 4 == 0 && a16(g.A) && a16(g.ln_g) && a16(g.ln_b) &&
           (!g.ln_out || a16(g.ln_out)) && (!g.a_add || (a16(g.a_add) && g.a_add_n % 32 == 0)) &&
           (int64_t)g.M * g.lda < 0x7fffffff && (int64_t)g.K * g.ldb < 0x7fffffff;
}

bool small16_ok(const GemmArgs &g, int amode);
hipError_t launch_small16(const GemmArgs &g, int amode, hipStream_t s);

hipError_t launch_ln(const GemmArgs &g, hipStream_t s) {
    if (!ln_ok(g)) return hipErrorInvalidValue;
    if (small16_ok(g, 1)) return launch_small16(g, 1, s);
    const int tiles_m = (g.M + 31) / 32, tiles_n = (g.N + 31) / 32, tmn = tiles_m * tiles_n;
    const dim3 grid((unsigned)tmn);
    const bool pre = g.a_add != nullptr;
    if (g.K == 8 * kSmallKC) {
        if (pre) hipLaunchKernelGGL((k_gemm_small_ln<8, true>), grid, dim3(512), 0, s, g, tiles_m, tmn);
        else hipLaunchKernelGGL((k_gemm_small_ln<8, false>), grid, dim3(512), 0, s, g, tiles_m, tmn);
    } else {
        if (pre) hipLaunchKernelGGL((k_gemm_small_ln<16, true>), grid, dim3(1024), 0, s, g, tiles_m, tmn);
        else hipLaunchKernelGGL((k_gemm_small_ln<16, false>), grid, dim3(1024), 0, s, g, tiles_m, tmn);
    }
    return hipGetLastError();
}

template <int BMODE>
hipError_t dispatch(const GemmArgs &g_in, const GemmWorkspace &ws, hipStream_t s) {
    GemmArgs g = g_in;
    g.n_vec = BMODE == 0 ? n_vec_of(g) : 0;
    if (g.ln_g) return BMODE == 0 ? launch_ln(g, s) : hipErrorInvalidValue;
    if (BMODE == 1) {
        if (const int cc = patch_cc(g)) return launch_patch(g, cc, s);
        if (direct_ok(g)) return launch_direct(g, s);
        if (k2q_ok(g)) return launch_k2q(g, s);
        if (k3s2q_ok(g)) return launch_k3s2q(g, s);
        if (frag_ok(g)) return launch_frag(g, s);
    }
    if (g.a_w4) {
        // A = relu(X W4 + b4): the small kernel's computed-A loader
        const auto a16 = [](const void *q) { return (((uintptr_t)q) & 15) == 0; };
        if (BMODE != 0 || !g.a_rowmajor || g.a_add || !g.a_b4 || g.lda != 4 || g.K % 4 != 0 || !a16(g.A) ||
            !a16(g.a_w4) || !a16(g.a_b4))
            return hipErrorInvalidValue;
        if (g.box_h) {
            // the box prologue exists in the 16 x 32 kernel only
            const bool box_ok = small16_ok(g, 2) && g.box_k == 256 && g.box_ldh % 4 == 0 && g.box_ldh >= 256 &&
                                a16(g.box_h) && a16(g.box_w) && g.box_b && g.box_out && a16(g.box_out) &&
                                (int64_t)g.M * g.box_ldh < 0x7fffffff;
            return box_ok ? launch_small16(g, 2, s) : hipErrorInvalidValue;
        }
        return launch_small<2>(g, s);
    }
    const GemmPlan p = gemm_plan(g, ws.bytes, BMODE == 1);
    if constexpr (BMODE == 0) {
        const int lc = gemm_lt_pick(g, 8 * cus_per_xcd(), lt_wanted(g, p));
        if (lc >= 0) return gemm_lt(g, lc, s);
    }
    if (g.a_add && (BMODE != 0 || !g.a_rowmajor || (((uintptr_t)g.a_add) & 15) != 0 || g.a_add_n % 32 != 0))
        return hipErrorInvalidValue;
    // sign-bit output: the tiled kernels' shared epilogue, whole 32-column words
    if (g.bits && (p.cfg == kCfgSmall || p.splits > 1 || g.c_trans || g.N % 32 != 0 || g.a_w4 || BMODE != 0))
        return hipErrorInvalidValue;
    if (BMODE == 0 && p.cfg == kCfgSmall) {
        if (g.a_rowmajor && (g.K % 4 != 0 || g.lda % 4 != 0 || (((uintptr_t)g.A) & 15) != 0))
            return hipErrorInvalidValue;
        return g.a_rowmajor ? launch_small<1>(g, s) : launch_small<0>(g, s);
    }
    if (g.a_rowmajor) {
        // row-major A (token-major activations) is built for the two block
        // shapes the planner uses
        if (BMODE != 0 || g.K % 4 != 0 || g.lda % 4 != 0 || (((uintptr_t)g.A) & 15) != 0)
            return hipErrorInvalidValue;
        if (p.cfg == 5) return launch<32, 128, 1, 1, 0>(g, p.splits, ws, s);
        return launch<64, 64, 2, 1, 0>(g, p.splits, ws, s);
    }
    if constexpr (BMODE == 1) {
        // IC >= kBK without one tap per k tile, or IC == kBK / 2 (every k tile
        // exactly two taps): the two-tap loader (64x64 or 32x128 blocks, the
        // shapes the im2col planner picks)
        if ((g.IC >= kBK && !(g.IC % kBK == 0 && g.K % kBK == 0)) || g.IC == kBK / 2) {
            if (p.cfg == 5) return launch<32, 128, 1, 0, 2>(g, p.splits, ws, s);
            if (p.cfg == 3) return launch<64, 64, 2, 0, 2>(g, p.splits, ws, s);
        }
    }
    switch (p.cfg) {
        case 0: return launch<128, 128, 2, 0, BMODE>(g, p.splits, ws, s);
        case 1: return launch<64, 128, 2, 0, BMODE>(g, p.splits, ws, s);
        case 2: return launch<128, 64, 2, 0, BMODE>(g, p.splits, ws, s);
        case 3: return launch<64, 64, 2, 0, BMODE>(g, p.splits, ws, s);
        case 4: return launch<32, 256, 1, 0, BMODE>(g, p.splits, ws, s);
        default: return launch<32, 128, 1, 0, BMODE>(g, p.splits, ws, s);
    }
}

}  // namespace

int64_t gemm_ws_bytes(int M, int N, int batch, int cfg, int splits) {
    (void)cfg;
    if (splits <= 1) return 0;
    return (int64_t)splits * batch * M * N * 4;
}

GemmPlan gemm_plan(const GemmArgs &g, int64_t ws_bytes, bool im2col) {
    GemmPlan best;
    int oc, os;
    const int nk = (g.K + kBK - 1) / kBK;
    if (env_override(&oc, &os)) {
        if (oc == kCfgSmall && im2col) oc = 3;  // the small kernel reads dense B only
        best.cfg = oc;
        best.splits = oc == kCfgSmall ? 1 : (os < nk ? os : nk);  // at most one split per k tile
    } else {
        best = plan_auto(g.M, g.N, g.K, g.batch, im2col);
    }
    // the prologue add exists in the small kernel only
    if (g.a_add && !im2col) best = GemmPlan{kCfgSmall, 1};
    // never plan more splits than the workspace holds
    while (best.splits > 1 && gemm_ws_bytes(g.M, g.N, g.batch, best.cfg, best.splits) > ws_bytes) best.splits--;
    return best;
}

int64_t gemm_ws_bytes_for(const GemmArgs &g, bool im2col) {
    if (g.a_w4 || g.ln_g) return 0;  // the small kernel, no split-K
    if (im2col && !patch_cc(g) && (direct_ok(g) || k2q_ok(g) || k3s2q_ok(g) || frag_ok(g))) return 0;  // no workspace
    const GemmPlan p = gemm_plan(g, INT64_MAX, im2col);
    return gemm_ws_bytes(g.M, g.N, g.batch, p.cfg, p.splits);
}

hipError_t gemm_dense(const GemmArgs &g, const GemmWorkspace &ws, hipStream_t s) { return dispatch<0>(g, ws, s); }

std::string gemm_kernel_name(const GemmArgs &g, int64_t ws_bytes, bool im2col) {
    if (im2col && patch_cc(g)) return g.KW == 3 ? "k_conv_patch<3, 2>" : "k_conv_patch<2, 1>";
    if (im2col && direct_ok(g)) return "k_conv_k3s2<" + std::to_string(g.IC) + ">";
    if (im2col && k2q_ok(g)) return "k_conv_k2q<" + std::to_string(g.IC) + (g.M <= 16 ? ", 1>" : ", 2>");
    if (im2col && k3s2q_ok(g)) return std::string("k_conv_k3s2q<64, ") + (g.M <= 16 ? "1>" : "2>");
    if (im2col && frag_ok(g)) return "k_conv_frag<" + std::to_string(frag_waves(g)) + ">";
    if (g.a_w4 && small16_ok(g, 2))
        return g.box_h ? "k_gemm_small16<3, 8, false, false>" : "k_gemm_small16<2, 8, false, false>";
    if (g.a_w4) return "k_gemm_small<2, " + std::to_string(small_waves(g.K, small_tiles(g))) + ", false>";

    const GemmPlan p = gemm_plan(g, ws_bytes, im2col);
    if (!im2col) {
        GemmArgs gv = g;
        gv.n_vec = n_vec_of(g);
        const int lc = gemm_lt_pick(gv, 8 * cus_per_xcd(), lt_wanted(gv, p));
        if (lc >= 0) return gemm_lt_name(lc);
    }
    if (g.a_rowmajor && (g.ln_g || p.cfg == kCfgSmall) && small16_ok(g, 1)) {
        const char *ew = getenv("PPDL_SMALL16_WV16");
        const bool w8 = g.ln_g || !(ew && ew[0] == '1');
        return std::string("k_gemm_small16<1, ") + (w8 ? "8, " : "16, ") + (g.ln_g ? "true, " : "false, ") +
               (g.a_add ? "true>" : "false>");
    }
    if (g.ln_g) return "k_gemm_small_ln<" + std::to_string(g.K / kSmallKC) + (g.a_add ? ", true>" : ", false>");
    if (p.cfg == kCfgSmall)
        return std::string("k_gemm_small<") + (g.a_rowmajor ? "1, " : "0, ") +
               std::to_string(small_waves(g.K, small_tiles(g))) + (g.a_add && g.a_rowmajor ? ", true>" : ", false>");
    int bm = kCfgs[p.cfg].bm, bn = kCfgs[p.cfg].bn, wgm = kCfgs[p.cfg].wgm;
    if (g.a_rowmajor && p.cfg != 5) bm = 64, bn = 64, wgm = 2;  // the two row-major-A shapes
    char buf[96];
    if (!im2col && dma_ok(g)) {
        const int kg = (kBK * bm / 4 >= 2 * kThreads && kBK * bn / 4 >= 2 * kThreads) ? dma_groups() : 1;
        const bool tail = kg == 2 && bm == 64 && bn == 64 && wgm == 2 && p.splits == 1 &&
                          tail_grid((int64_t)((g.M + 63) / 64) * ((g.N + 63) / 64) * g.batch) > 0;
        snprintf(buf, sizeof(buf), "k_gemm_dma<%d, %d, %d, %s, 2, %d, %s>%s", bm, bn, wgm,
                 p.splits > 1 ? "true" : "false", kg, tail ? "true" : "false", p.splits > 1 ? "+k_splitk_reduce" : "");
    } else {
        const bool two_tap = im2col && ((g.IC >= kBK && !(g.IC % kBK == 0 && g.K % kBK == 0)) || g.IC == kBK / 2) &&
                             (p.cfg == 3 || p.cfg == 5);
        snprintf(buf, sizeof(buf), "k_gemm<%d, %d, %d, %d, %d, %s>%s", bm, bn, wgm, g.a_rowmajor ? 1 : 0,
                 two_tap ? 2 : im2col ? 1 : 0, p.splits > 1 ? "true" : "false", p.splits > 1 ? "+k_splitk_reduce" : "");
    }
    return buf;
}
hipError_t gemm_im2col(const GemmArgs &g, const GemmWorkspace &ws, hipStream_t s) { return dispatch<1>(g, ws, s); }

}  // namespace ppdl
