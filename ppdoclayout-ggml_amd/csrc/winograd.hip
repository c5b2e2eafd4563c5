// Winograd F(4,3) transforms for k3 s1 p1 convs (ops 10, 11, 15).
//
// Pipeline (same three-node split as patches/ggml-ppdl.patch:496-610, :778-812):
//   input  : dt[p][ic][t] = (Bt d Bt^T)[p]   d = 6x6 patch of tile t, stride 4
//   madd   : yt[p][oc][t] = sum_ic dt[p][ic][t] * wg4[p][ic][oc]   (gemm_f32)
//   output : y[oc][4ty+i][4tx+j] = act( (At m At^T)[i][j] + bias[oc] )
// with this library's own matrices (ppdl_internal.h).  Tiles are row-major
// over a TW x TH grid; the 36 planes are p = u*6 + v.
//
// Both transforms are HBM-bound: one thread per (channel, tile), consecutive
// threads on consecutive tiles, so every plane store (input transform) and
// every plane load (output transform) is a contiguous run along t.  A plane
// row (one channel's T tiles) may be padded to a stride ldt >= T; the
// padding is never written by the input transform nor read by the output.  The
// arithmetic is a fixed chain of fmaf over the nonzero matrix entries in
// ascending index order, which the CPU oracle repeats exactly.
#include <cstdlib>
#include <string>

#include "device_math.h"

namespace ppdl {
namespace {

constexpr int kThreads = 256;
constexpr int kChainRows = 8;  // tile rows per band of the chained transforms

// v = Bt d Bt^T of one 6x6 patch, plane p = u*6 + v: a fixed chain of fmaf
// over the nonzero entries in ascending index order (the oracle repeats it)
__device__ __forceinline__ void input_tile(const float (&d)[6][6], float (&out)[36]) {
    float t1[6][6];
#pragma unroll
    for (int u = 0; u < 6; u++)
#pragma unroll
        for (int b = 0; b < 6; b++) {
            float s = 0.0f;
#pragma unroll
            for (int a = 0; a < 6; a++)
                if (kBt[u][a] != 0.0f) s = fmaf(kBt[u][a], d[a][b], s);
            t1[u][b] = s;
        }
#pragma unroll
    for (int u = 0; u < 6; u++)
#pragma unroll
        for (int v = 0; v < 6; v++) {
            float s = 0.0f;
#pragma unroll
            for (int b = 0; b < 6; b++)
                if (kBt[v][b] != 0.0f) s = fmaf(t1[u][b], kBt[v][b], s);
            out[u * 6 + v] = s;
        }
}

// Y = At m At^T (4x4) of one tile's 36 plane values m[u][v]
__device__ __forceinline__ void output_tile(const float (&m)[6][6], float (&Y)[4][4]) {
    float t1[4][6];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int v = 0; v < 6; v++) {
            float s = 0.0f;
#pragma unroll
            for (int u = 0; u < 6; u++)
                if (kAt[i][u] != 0.0f) s = fmaf(kAt[i][u], m[u][v], s);
            t1[i][v] = s;
        }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < 6; v++)
                if (kAt[j][v] != 0.0f) s = fmaf(t1[i][v], kAt[j][v], s);
            Y[i][j] = s;
        }
}

// PAD = 0: x is the padded image (IWp x IHp), tile (ty,tx) reads rows 4ty..4ty+5.
// PAD = 1: x is the unpadded image, the conv's pad of 1 is applied on the fly.
template <int PAD>
__global__ __launch_bounds__(kThreads) void k_wg4_input(const float *__restrict__ x,
                                                        float *__restrict__ dt, int IW, int IH,
                                                        int IC, int TW, int TH, int ldt, int vec) {
    const int T = TW * TH;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= (int64_t)T * IC) return;
    const int ic = (int)(idx / T);
    const int tile = (int)(idx - (int64_t)ic * T);
    const int ty = tile / TW, tx = tile - ty * TW;
    const float *__restrict__ xc = x + (int64_t)ic * IH * IW;

    float d[6][6];
    if (PAD && vec) {
        // rows as one aligned float4 (columns 4tx .. 4tx+3, inside the row:
        // the host sets vec only for IW % 4 == 0 and a 16-byte aligned x)
        // plus the two halo columns: 18 loads, not 36.
        // Out-of-image rows / columns read a clamped in-image address and are
        // zeroed by select.
        const bool left = tx > 0, right = 4 * tx + 4 < IW;
#pragma unroll
        for (int a = 0; a < 6; a++) {
            const int iy = 4 * ty - 1 + a;
            const bool rin = iy >= 0 && iy < IH;
            const float *row = xc + (int64_t)min(max(iy, 0), IH - 1) * IW + 4 * tx;
            const float4 v = *reinterpret_cast<const float4 *>(row);
            const float l = row[left ? -1 : 0], r = row[right ? 4 : 3];
            d[a][0] = rin && left ? l : 0.0f;
            d[a][1] = rin ? v.x : 0.0f;
            d[a][2] = rin ? v.y : 0.0f;
            d[a][3] = rin ? v.z : 0.0f;
            d[a][4] = rin ? v.w : 0.0f;
            d[a][5] = rin && right ? r : 0.0f;
        }
    } else {
#pragma unroll
        for (int a = 0; a < 6; a++) {
            const int iy = 4 * ty - PAD + a;
#pragma unroll
            for (int b = 0; b < 6; b++) {
                const int ix = 4 * tx - PAD + b;
                if (PAD) {
                    d[a][b] = (iy >= 0 && iy < IH && ix >= 0 && ix < IW) ? xc[(int64_t)iy * IW + ix] : 0.0f;
                } else {
                    d[a][b] = xc[(int64_t)iy * IW + ix];
                }
            }
        }
    }
    float v[36];
    input_tile(d, v);
    float *__restrict__ o = dt + (int64_t)ic * ldt + tile;
    const int64_t pstride = (int64_t)IC * ldt;
#pragma unroll
    for (int p = 0; p < 36; p++) o[p * pstride] = v[p];
}

// add (optional, out's shape): a map added after the activation.  ACT: the
// activation code fixed at compile time for the common ones (-1: runtime).
template <int ACT>
__global__ __launch_bounds__(kThreads) void k_wg4_output(const float *__restrict__ yt,
                                                         const float *__restrict__ bias,
                                                         const float *__restrict__ add,
                                                         float *__restrict__ out, int TW, int TH,
                                                         int OC, int OW, int OH, int act, int ldt) {
    const int T = TW * TH;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= (int64_t)T * OC) return;
    const int oc = (int)(idx / T);
    const int tile = (int)(idx - (int64_t)oc * T);
    const int ty = tile / TW, tx = tile - ty * TW;

    const float *__restrict__ src = yt + (int64_t)oc * ldt + tile;
    const int64_t pstride = (int64_t)OC * ldt;
    float m[6][6];
#pragma unroll
    for (int p = 0; p < 36; p++) m[p / 6][p % 6] = src[p * pstride];

    float Y[4][4];
    output_tile(m, Y);
    const float b = bias[oc];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) Y[i][j] = act_t<ACT>(Y[i][j] + b, act);

    float *__restrict__ oplane = out + (int64_t)oc * OH * OW;
    const float *__restrict__ aplane = add ? add + (int64_t)oc * OH * OW : nullptr;
    const int px = 4 * tx;
    const bool vec = ((OW & 3) == 0) && ((((uintptr_t)out | (uintptr_t)add) & 15) == 0) && (px + 3 < OW);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int py = 4 * ty + i;
        if (py < OH) {
            float *row = oplane + (int64_t)py * OW + px;
            const float *arow = aplane ? aplane + (int64_t)py * OW + px : nullptr;
            if (vec) {
                float4 v = make_float4(Y[i][0], Y[i][1], Y[i][2], Y[i][3]);
                if (arow) {
                    const float4 a = *reinterpret_cast<const float4 *>(arow);
                    v.x += a.x, v.y += a.y, v.z += a.z, v.w += a.w;
                }
                *reinterpret_cast<float4 *>(row) = v;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (px + j < OW) row[j] = arow ? Y[i][j] + arow[j] : Y[i][j];
            }
        }
    }
}


// ---------------------------------------------------------------------------
// Chained transforms: the output transform of conv i (+ bias + act, its map
// y stored) and the input transform (pad 1) of conv i+1 on that map in one
// kernel, so y is not read back from memory and one launch disappears.
// A block owns a band of RB tile rows x all TW tile columns for CB channels:
//   1. output tiles of rows ty0 - 1 .. ty0 + RB (one halo row above and
//      below, recomputed by the neighbouring bands too) into an LDS image of
//      the band with a one-pixel frame; pixels outside the map are zero (the
//      next conv's padding); the band's own rows are also stored to y;
//   2. input transforms of the band's tiles from the LDS image, stored to
//      dt [36][C][ldt_in] like op 15.
// LDS row k holds map row 4 (ty0 - 1) + k, LDS column k map column k - 1.
template <int CB>
__global__ __launch_bounds__(kThreads) void k_wg4_chain(const float *__restrict__ yt, const float *__restrict__ bias,
                                                        float *__restrict__ y, float *__restrict__ dt, int TW, int TH,
                                                        int C, int OW, int OH, int act, int ldt_out, int ldt_in) {
    constexpr int RB = kChainRows;
    extern __shared__ float band[];  // [CB][LH][LW]
    const int LW = 4 * TW + 2, LH = 4 * (RB + 2);
    const int nb = (TH + RB - 1) / RB;
    const int ty0 = (int)(blockIdx.x % nb) * RB, c0 = (int)(blockIdx.x / nb) * CB;
    const int64_t pout = (int64_t)C * ldt_out, pin = (int64_t)C * ldt_in;

    // frame columns (map columns -1 and 4 TW): zero
    for (int i = threadIdx.x; i < CB * LH; i += kThreads) {
        band[i * LW] = 0.0f;
        band[i * LW + LW - 1] = 0.0f;
    }
    const int n1 = CB * (RB + 2) * TW;
    for (int task = threadIdx.x; task < n1; task += kThreads) {
        const int cc = task / ((RB + 2) * TW), r = task - cc * ((RB + 2) * TW);
        const int tyl = r / TW, tx = r - tyl * TW;
        const int ty = ty0 - 1 + tyl, c = c0 + cc;
        const bool live = ty >= 0 && ty < TH && c < C;
        float Y[4][4];
        if (live) {
            const float *src = yt + (int64_t)c * ldt_out + ty * TW + tx;
            float m[6][6];
#pragma unroll
            for (int p = 0; p < 36; p++) m[p / 6][p % 6] = src[p * pout];
            output_tile(m, Y);
            const float b = bias[c];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) Y[i][j] = act_f(Y[i][j] + b, act);
        }
        float *lrow = band + ((int64_t)cc * LH + 4 * tyl) * LW + 1 + 4 * tx;
        const bool own = live && tyl >= 1 && tyl <= RB;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int py = 4 * ty + i;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int px = 4 * tx + j;
                const bool in = live && py < OH && px < OW;
                lrow[i * LW + j] = in ? Y[i][j] : 0.0f;
                if (own && in) y[((int64_t)c * OH + py) * OW + px] = Y[i][j];
            }
        }
    }
    __syncthreads();
    const int n2 = CB * RB * TW;
    for (int task = threadIdx.x; task < n2; task += kThreads) {
        const int cc = task / (RB * TW), r = task - cc * (RB * TW);
        const int tyl = r / TW, tx = r - tyl * TW;
        const int ty = ty0 + tyl, c = c0 + cc;
        if (ty >= TH || c >= C) continue;
        // patch rows: map rows 4 ty - 1 + a = LDS rows 4 tyl + 3 + a; columns
        // 4 tx - 1 + b = LDS columns 4 tx + b
        const float *l = band + ((int64_t)cc * LH + 4 * tyl + 3) * LW + 4 * tx;
        float d[6][6];
#pragma unroll
        for (int a = 0; a < 6; a++)
#pragma unroll
            for (int b = 0; b < 6; b++) d[a][b] = l[a * LW + b];
        float v[36];
        input_tile(d, v);
        float *o = dt + (int64_t)c * ldt_in + ty * TW + tx;
#pragma unroll
        for (int p = 0; p < 36; p++) o[p * pin] = v[p];
    }
}


// ---------------------------------------------------------------------------
// Fused F(4,3) conv (op 17): input transform, the 36 per-plane channel
// contractions and output transform + bias + act in one kernel; the dt / yt
// planes never reach memory.
//
// A block of 6 waves owns 16 tiles (raster order) x 16*OT output channels and
// walks the input channels 4 at a time (one "step").  Per step:
//   * column stage: thread (wave b, lane l = 16 q + c) loads column b of the
//     6x6 patch of channel ic0 + q around tile t0 + c and forms column b of
//     Bt d (the input transform's first fmaf chains), into LDS;
//   * the step's weights wg4[p][ic0 .. ic0+3][oc0 .. oc0+16*OT) are copied to
//     LDS with float4 loads;
//   * row stage: wave u finishes row u of Bt d Bt^T for its lane's (channel,
//     tile) (the second fmaf chains): 6 values that are exactly its B operand
//     (k = q, n = c) of planes 6u .. 6u+5, and runs those planes' products
//     with v_mfma_f32_16x16x4f32 against the weights from LDS (A operand
//     m = c, k = q), OT channel tiles per plane; register r of an
//     accumulator holds (channel oc0 + 16 o + 4 q + r, tile t0 + c).
// Operands of step s + 1 are loaded into registers before the row stage of
// step s; LDS is double-buffered, so one barrier per step orders the stages.
// After the last step wave u reduces its row: z_u[j] = sum_v M[u][v] At[j][v]
// per (channel, tile), to LDS; then each thread finishes whole pairs,
// Y[i][j] = sum_u At[i][u] z_u[j], adds the bias, applies the activation and
// stores the 4x4 output tile.  Channels past IC get zero patches and zero
// weights.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int OT, bool VW, bool FULL>
__global__ __launch_bounds__(384) void k_wg4_conv(const float *__restrict__ x, const float *__restrict__ wg4,
                                                 const float *__restrict__ bias, float *__restrict__ out, int IC,
                                                 int H, int W, int OC, int TW, int T, int act, int nocb, int vout) {
    constexpr int OCB = 16 * OT;                  // channels per block
    constexpr int T1F = 36 * 64;                  // floats of one step's column stage
    constexpr int A4 = 36 * 4 * OCB / 4;          // float4s of one step's weights
    constexpr int AL = (A4 + 383) / 384;          // float4 loads per thread
    constexpr int AF = AL * 384 * 4;              // LDS floats per weight buffer (a pad takes the excess)
    constexpr int ZF = 6 * 4 * OCB * 16;          // floats of the final row sums (6 rows x 4 j x pairs)
    constexpr int SMEM = (2 * (T1F + AF) > ZF) ? 2 * (T1F + AF) : ZF;
    constexpr int D = 3;                          // steps of loads in flight
    __shared__ __attribute__((aligned(16))) float smem[SMEM];
    float *const T1s = smem;             // [2][6 u][6 b][64 lanes]
    float *const As = smem + 2 * T1F;    // [2][36 p][4 k][OCB]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, q = lane >> 4;
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    const int ocb = blk % nocb, tg = blk / nocb;
    const int oc0 = ocb * OCB, t0 = tg * 16;
    const int plane = H * W;
    const int nsteps = (IC + 3) >> 2;

    // column stage geometry: this thread's patch column b = wave of the tile
    // t0 + c (a tile past T repeats tile T - 1; it is not stored)
    const int t = t0 + c;
    const int tc = t < T ? t : T - 1;
    const int ty = tc / TW, tx = tc - ty * TW;
    const int ix = 4 * tx - 1 + wave;
    const bool col_in = ix >= 0 && ix < W;
    const int ixc = min(max(ix, 0), W - 1);

    // Per-thread load geometry, fixed for the whole channel walk: the patch
    // column's 6 row offsets (clamped) and in-image mask, and for each of the
    // thread's weight float4s its plane / channel-in-step / channel-quad
    // offsets.  Offsets are 32-bit (the host checks the extents).
    int prow[6];
    uint32_t rowm = 0;
#pragma unroll
    for (int r = 0; r < 6; r++) {
        const int iy = 4 * ty - 1 + r;
        prow[r] = min(max(iy, 0), H - 1) * W + ixc;
        rowm |= (col_in && iy >= 0 && iy < H) ? (1u << r) : 0u;
    }
    int wbase[AL], wk[AL], wlim[AL];
    uint32_t wm = 0;  // bit j: weight float4 j inside the step's table and OC
#pragma unroll
    for (int j = 0; j < AL; j++) {
        const int e = tid + j * 384;
        const int ee = min(e, A4 - 1);
        const int quad = ee % (OCB / 4), pk = ee / (OCB / 4);
        const int ocw = oc0 + 4 * quad;
        const int occ = VW ? min(ocw, OC - 4) : min(ocw, OC - 1);
        wk[j] = pk & 3;
        wbase[j] = (pk >> 2) * IC * OC + occ;
        wlim[j] = OC - 1 - occ;  // channels after the quad's first, within the row (scalar path)
        wm |= (e < A4 && ocw < OC) ? (1u << j) : 0u;
    }
    const int last = nsteps - 1;

    // Loads of one step go to registers unmasked (clamped, always-valid
    // addresses; steps past the last repeat it); the masks are applied when
    // the step is stored to LDS, so the loads never depend on a condition.
    struct Pre {
        float d[6];
        float4 a[AL];
        uint32_t m;  // bits 0-5: patch rows inside; bit 6 + j: weight float4 j inside
    };
    auto load = [&](Pre &pr, int su) {
        // su past the last step: clamped addresses, all masks clear, so the
        // step adds exact zeros
        const int st = min(su, last);
        const int ic = 4 * st + q, icu = 4 * su + q;
        // 32-bit element offsets from the kernel-argument bases (uniform base
        // + 32-bit lane offset: no 64-bit address per load kept live)
        const uint32_t xo = (uint32_t)(min(ic, IC - 1) * plane);
#pragma unroll
        for (int r = 0; r < 6; r++) pr.d[r] = x[xo + (uint32_t)prow[r]];
        uint32_t m = icu < IC ? rowm : 0u;
#pragma unroll
        for (int j = 0; j < AL; j++) {
            const int icw = 4 * su + wk[j];
            const float *src = wg4 + (uint32_t)(wbase[j] + min(4 * st + wk[j], IC - 1) * OC);
            if (VW) {
                pr.a[j] = *reinterpret_cast<const float4 *>(src);
            } else {
                pr.a[j].x = src[0];
                pr.a[j].y = src[min(1, wlim[j])];
                pr.a[j].z = src[min(2, wlim[j])];
                pr.a[j].w = src[min(3, wlim[j])];
            }
            if (!FULL) m |= (((wm >> j) & 1u) && icw < IC) ? (1u << (6 + j)) : 0u;
        }
        pr.m = m;
    };
    // column stage of a prefetched step into LDS buffer `buf`
    auto store = [&](const Pre &pr, int buf) {
        float d[6];
#pragma unroll
        for (int r = 0; r < 6; r++) d[r] = ((pr.m >> r) & 1u) ? pr.d[r] : 0.0f;
        float *t1 = T1s + buf * T1F + wave * 64 + lane;  // [u][b = wave][lane]
#pragma unroll
        for (int uu = 0; uu < 6; uu++) {
            float sum = 0.0f;
#pragma unroll
            for (int a = 0; a < 6; a++)
                if (kBt[uu][a] != 0.0f) sum = fmaf(kBt[uu][a], d[a], sum);
            t1[uu * 6 * 64] = sum;
        }
        float4 *as = reinterpret_cast<float4 *>(As + buf * AF);
#pragma unroll
        for (int j = 0; j < AL; j++) {
            const int e = tid + j * 384;
            const int quad = min(e, A4 - 1) % (OCB / 4);
            const int ocw = oc0 + 4 * quad;
            float4 v = pr.a[j];
            // FULL: every step inside IC, every quad inside OC (a float4 past
            // the table lands in the pad), so no weight needs masking
            const bool in = FULL || ((pr.m >> (6 + j)) & 1u);
            v.x = in ? v.x : 0.0f;
            v.y = (in && (VW || ocw + 1 < OC)) ? v.y : 0.0f;
            v.z = (in && (VW || ocw + 2 < OC)) ? v.z : 0.0f;
            v.w = (in && (VW || ocw + 3 < OC)) ? v.w : 0.0f;
            as[e] = v;  // e >= A4 lands in the pad
        }
    };

    f32x4 acc[OT][6];
#pragma unroll
    for (int o = 0; o < OT; o++)
#pragma unroll
        for (int v = 0; v < 6; v++) acc[o][v] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int u = wave;  // this wave's plane row in the row stage

    // Prefetch ring: slot k holds the step congruent to k mod D.  Iteration s
    // runs the row stage of step s, stores step s + 1 (loaded D - 1
    // iterations earlier) into the other LDS buffer and reloads that slot
    // with step s + 1 + D.  The loop is unrolled by D so slots are registers,
    // and it runs whole groups of D steps (the steps past the last add
    // zeros), so the loop has no exit between the unrolled steps.
    Pre pre[D];
#pragma unroll
    for (int k = 0; k < D; k++) load(pre[k], k);
    store(pre[0], 0);
    load(pre[0], D);
    for (int s0 = 0; s0 < nsteps; s0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int st = s0 + k;
            const int buf = st & 1;
            __syncthreads();  // step st's column stage and weights are in LDS
            // row stage
            const float *t1 = T1s + buf * T1F + u * 6 * 64 + lane;
            float tr[6];
#pragma unroll
            for (int b = 0; b < 6; b++) tr[b] = t1[b * 64];
            float vv[6];
#pragma unroll
            for (int v = 0; v < 6; v++) {
                float sum = 0.0f;
#pragma unroll
                for (int b = 0; b < 6; b++)
                    if (kBt[v][b] != 0.0f) sum = fmaf(tr[b], kBt[v][b], sum);
                vv[v] = sum;
            }
            const float *as = As + buf * AF + (u * 6 * 4 + q) * OCB + c;  // [p = 6u + v][k = q][16 o + c]
#pragma unroll
            for (int v = 0; v < 6; v++)
#pragma unroll
                for (int o = 0; o < OT; o++)
                    acc[o][v] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(as[v * 4 * OCB + 16 * o], vv[v], acc[o][v], 0, 0, 0);
            // step st + 1 into the other buffer (its last readers passed this
            // step's barrier; past the last step a repeat nobody reads), then
            // its slot takes step st + 1 + D
            const int kn = (k + 1) % D;  // a constant once the loop is unrolled
            store(pre[kn], buf ^ 1);
            load(pre[kn], st + 1 + D);
        }
    }
    __syncthreads();  // every row stage is done before LDS is reused

    // row u's share of the output transform: z[o][r][j] = sum_v M[u][v] At[j][v]
    // for the lane's pairs (channel oc0 + 16 o + 4 q + r, tile t0 + c)
    float *Z = smem;  // [u][j][pair], pair = (16 o + 4 q + r) * 16 + c
#pragma unroll
    for (int o = 0; o < OT; o++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float sum = 0.0f;
#pragma unroll
                for (int v = 0; v < 6; v++)
                    if (kAt[j][v] != 0.0f) sum = fmaf(acc[o][v][r], kAt[j][v], sum);
                Z[(u * 4 + j) * (OCB * 16) + (16 * o + 4 * q + r) * 16 + c] = sum;
            }
    __syncthreads();
    const int px = 4 * tx;  // (thread-specific below)
    (void)px;
    for (int pr = tid; pr < OCB * 16; pr += 384) {
        const int ocl = pr >> 4, cc = pr & 15;
        const int oc = oc0 + ocl, tt = t0 + cc;
        if (oc >= OC || tt >= T) continue;
        float z[6][4];
#pragma unroll
        for (int uu = 0; uu < 6; uu++)
#pragma unroll
            for (int j = 0; j < 4; j++) z[uu][j] = Z[(uu * 4 + j) * (OCB * 16) + pr];
        const int oty = tt / TW, otx = tt - oty * TW;
        const float b = bias[oc];
        float *__restrict__ oplane = out + (int64_t)oc * plane;
        const int ox = 4 * otx;
        const bool vec = vout && ox + 3 < W;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int py = 4 * oty + i;
            if (py >= H) continue;
            float y[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float sum = 0.0f;
#pragma unroll
                for (int uu = 0; uu < 6; uu++)
                    if (kAt[i][uu] != 0.0f) sum = fmaf(kAt[i][uu], z[uu][j], sum);
                y[j] = act_f(sum + b, act);
            }
            float *row = oplane + (int64_t)py * W + ox;
            if (vec) {
                *reinterpret_cast<float4 *>(row) = make_float4(y[0], y[1], y[2], y[3]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (ox + j < W) row[j] = y[j];
            }
        }
    }
}

}  // namespace

// Channel tiles of 16 per block of the fused conv: all of them (one block
// per tile group) up to 48 output channels, else 1 (measured on the
// network's shapes: 48 -> 48 @200 runs 28.8 us with 3 tiles against 31.8
// with 1; 96 -> 96 @100 and 64 -> 64 @100 are fastest with 1).  PPDL_WG_OT
// pins 1 .. 4 (sweeps and tests).
int wg4_conv_ot(int IC, int H, int W, int OC) {
    (void)IC;
    (void)H;
    (void)W;
    if (const char *e = getenv("PPDL_WG_OT")) {
        const int v = atoi(e);
        if (v >= 1 && v <= 4) return v;
    }
    const int tiles16 = (OC + 15) / 16;
    return tiles16 <= 3 ? tiles16 : 1;
}

std::string wg4_conv_kernel_name(int IC, int H, int W, int OC) {
    return "k_wg4_conv<" + std::to_string(wg4_conv_ot(IC, H, W, OC)) + ">";
}

hipError_t wg4_conv(const float *x, const float *wg4, const float *bias, float *out, int IC, int H, int W, int OC,
                    int act, hipStream_t s) {
    const int TW = (W + 3) / 4, TH = (H + 3) / 4, T = TW * TH;
    const int ot = wg4_conv_ot(IC, H, W, OC);
    const int nocb = (OC + 16 * ot - 1) / (16 * ot);
    const int64_t blocks = (int64_t)nocb * ((T + 15) / 16);
    if (blocks < 1 || blocks > 0x7fffffff || IC < 1 || OC < 1) return hipErrorInvalidValue;
    // the kernel's input and weight offsets are 32-bit
    if ((int64_t)IC * H * W > 0x7fffffff || (int64_t)36 * IC * OC > 0x7fffffff) return hipErrorInvalidValue;
    const bool vw = OC % 4 == 0 && (((uintptr_t)wg4) & 15) == 0;
    // no weight masks: whole 4-channel steps in whole groups of the kernel's
    // 3-step prefetch ring, whole channel tiles per block
    const int nsteps = (IC + 3) / 4;
    const bool full = vw && IC % 4 == 0 && nsteps % 3 == 0 && OC % (16 * ot) == 0;
    const int vout = (W % 4 == 0 && (((uintptr_t)out) & 15) == 0) ? 1 : 0;
    const dim3 grid((unsigned)blocks), blk(384);
#define PPDL_WG_LAUNCH(O)                                                                                        \
    do {                                                                                                         \
        if (full)                                                                                                \
            hipLaunchKernelGGL((k_wg4_conv<O, true, true>), grid, blk, 0, s, x, wg4, bias, out, IC, H, W, OC, TW, T, \
                               act, nocb, vout);                                                                 \
        else if (vw)                                                                                             \
            hipLaunchKernelGGL((k_wg4_conv<O, true, false>), grid, blk, 0, s, x, wg4, bias, out, IC, H, W, OC, TW, \
                               T, act, nocb, vout);                                                              \
        else                                                                                                     \
            hipLaunchKernelGGL((k_wg4_conv<O, false, false>), grid, blk, 0, s, x, wg4, bias, out, IC, H, W, OC, TW, \
                               T, act, nocb, vout);                                                              \
    } while (0)
    switch (ot) {
        case 1: PPDL_WG_LAUNCH(1); break;
        case 2: PPDL_WG_LAUNCH(2); break;
        case 3: PPDL_WG_LAUNCH(3); break;
        default: PPDL_WG_LAUNCH(4); break;
    }
#undef PPDL_WG_LAUNCH
    return hipGetLastError();
}

hipError_t wg4_input(const float *x, float *dt, int IW, int IH, int IC, int TW, int TH, int pad, int ldt,
                     hipStream_t s) {
    const int64_t n = (int64_t)TW * TH * IC;
    const unsigned blocks = (unsigned)((n + kThreads - 1) / kThreads);
    const int vec = (IW % 4 == 0 && (((uintptr_t)x) & 15) == 0) ? 1 : 0;
    if (pad)
        hipLaunchKernelGGL(k_wg4_input<1>, dim3(blocks), dim3(kThreads), 0, s, x, dt, IW, IH, IC, TW, TH, ldt, vec);
    else
        hipLaunchKernelGGL(k_wg4_input<0>, dim3(blocks), dim3(kThreads), 0, s, x, dt, IW, IH, IC, TW, TH, ldt, 0);
    return hipGetLastError();
}

bool wg4_chain_fits(int OW) {
    return (size_t)2 * 4 * (kChainRows + 2) * (4 * ((OW + 3) / 4) + 2) * sizeof(float) <= 64 * 1024;
}

hipError_t wg4_chain(const float *yt, const float *bias, float *y, float *dt, int C, int OW, int OH, int act,
                     int ldt_out, int ldt_in, hipStream_t s) {
    const int TW = (OW + 3) / 4, TH = (OH + 3) / 4, T = TW * TH;
    const int nb = (TH + kChainRows - 1) / kChainRows;
    if (C < 1 || OW < 1 || OH < 1 || ldt_out < T || ldt_in < T) return hipErrorInvalidValue;
    // 4 channels per block when that still gives 256 blocks and fits 64 KB
    // of LDS, else 2
    const size_t per_c = (size_t)4 * (kChainRows + 2) * (4 * TW + 2) * sizeof(float);
    const int cb = ((int64_t)nb * ((C + 3) / 4) >= 256 && 4 * per_c <= 64 * 1024) ? 4 : 2;
    const size_t lds = cb * per_c;
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)(nb * ((C + cb - 1) / cb));
    if (cb == 4)
        hipLaunchKernelGGL(k_wg4_chain<4>, dim3(blocks), dim3(kThreads), lds, s, yt, bias, y, dt, TW, TH, C, OW, OH,
                           act, ldt_out, ldt_in);
    else
        hipLaunchKernelGGL(k_wg4_chain<2>, dim3(blocks), dim3(kThreads), lds, s, yt, bias, y, dt, TW, TH, C, OW, OH,
                           act, ldt_out, ldt_in);
    return hipGetLastError();
}

hipError_t wg4_output(const float *yt, const float *bias, const float *add, float *out, int TW, int TH, int OC,
                      int OW, int OH, int act, int ldt, hipStream_t s) {
    const int64_t n = (int64_t)TW * TH * OC;
    const unsigned blocks = (unsigned)((n + kThreads - 1) / kThreads);
    switch (act) {
        case kActNone:
            hipLaunchKernelGGL(k_wg4_output<kActNone>, dim3(blocks), dim3(kThreads), 0, s, yt, bias, add, out, TW, TH,
                               OC, OW, OH, act, ldt);
            break;
        case kActSilu:
            hipLaunchKernelGGL(k_wg4_output<kActSilu>, dim3(blocks), dim3(kThreads), 0, s, yt, bias, add, out, TW, TH,
                               OC, OW, OH, act, ldt);
            break;
        default:
            hipLaunchKernelGGL(k_wg4_output<-1>, dim3(blocks), dim3(kThreads), 0, s, yt, bias, add, out, TW, TH, OC,
                               OW, OH, act, ldt);
            break;
    }
    return hipGetLastError();
}

}  // namespace ppdl
