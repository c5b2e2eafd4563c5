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
#include "device_math.h"

namespace ppdl {
namespace {

constexpr int kThreads = 256;

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
    float *__restrict__ o = dt + (int64_t)ic * ldt + tile;
    const int64_t pstride = (int64_t)IC * ldt;
#pragma unroll
    for (int u = 0; u < 6; u++)
#pragma unroll
        for (int v = 0; v < 6; v++) {
            float s = 0.0f;
#pragma unroll
            for (int b = 0; b < 6; b++)
                if (kBt[v][b] != 0.0f) s = fmaf(t1[u][b], kBt[v][b], s);
            o[(u * 6 + v) * pstride] = s;
        }
}

__global__ __launch_bounds__(kThreads) void k_wg4_output(const float *__restrict__ yt,
                                                         const float *__restrict__ bias,
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
    const float b = bias[oc];
    float Y[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < 6; v++)
                if (kAt[j][v] != 0.0f) s = fmaf(t1[i][v], kAt[j][v], s);
            Y[i][j] = act_f(s + b, act);
        }

    float *__restrict__ oplane = out + (int64_t)oc * OH * OW;
    const int px = 4 * tx;
    const bool vec = ((OW & 3) == 0) && ((((uintptr_t)out) & 15) == 0) && (px + 3 < OW);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int py = 4 * ty + i;
        if (py < OH) {
            float *row = oplane + (int64_t)py * OW + px;
            if (vec) {
                *reinterpret_cast<float4 *>(row) = make_float4(Y[i][0], Y[i][1], Y[i][2], Y[i][3]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (px + j < OW) row[j] = Y[i][j];
            }
        }
    }
}

}  // namespace

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

hipError_t wg4_output(const float *yt, const float *bias, float *out, int TW, int TH, int OC,
                      int OW, int OH, int act, int ldt, hipStream_t s) {
    const int64_t n = (int64_t)TW * TH * OC;
    const unsigned blocks = (unsigned)((n + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(k_wg4_output, dim3(blocks), dim3(kThreads), 0, s, yt, bias, out, TW, TH, OC,
                       OW, OH, act, ldt);
    return hipGetLastError();
}

}  // namespace ppdl
