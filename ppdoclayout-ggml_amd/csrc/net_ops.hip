// Stock ops of the PP-DocLayoutV3 graph that are not tagged ops: the work the
// reference leaves to ggml's own kernels (depthwise conv, pooling,
// interpolation, layer norm, attention, elementwise), written for gfx950.
// Semantics follow the ggml ops the reference graph calls
// (src/ppdoclayout.cpp:363-883); each kernel cites its call site.
#include <algorithm>

#include "device_math.h"
#include "net_internal.h"

#pragma clang fp contract(off)

namespace ppdl {
namespace {

// ---------------------------------------------------------------------------
// Depthwise conv + bias + act (ggml_conv_2d_dw_direct + add + act,
// src/ppdoclayout.cpp:400-404).  w: [C][K][K].  A block owns one channel and
// a band of RB output rows: it stages the band's input rows, zero-padded by P
// on every side, in LDS with coalesced loads, then each thread sums the K*K
// taps of its outputs in (kh, kw) order from LDS (K is a template argument:
// the taps are unrolled and their reads issued together).  A padding tap adds
// fmaf(0, w, s) = s, so the sum equals the one over in-bounds taps only.
// Bands are sized for ~2048 blocks so that enough waves hide LDS latency.
constexpr int kDwLds = 8192;  // floats of staged input per block

template <int K>
__global__ __launch_bounds__(256) void k_dwconv(const float *__restrict__ x, const float *__restrict__ w,
                                                const float *__restrict__ b, float *__restrict__ out, int C,
                                                int IH, int IW, int OH, int OW, int S, int P, int act, int RB,
                                                int64_t in_plane, int64_t out_plane) {
    __shared__ float tile[kDwLds];
    const int c = blockIdx.y, oy0 = blockIdx.x * RB;
    const int rows = min(RB, OH - oy0);
    const int TR = (rows - 1) * S + K, TC = IW + 2 * P;  // staged rows / columns
    const int iy0 = oy0 * S - P;
    const float *__restrict__ xc = x + (int64_t)c * in_plane;
    for (int i = threadIdx.x; i < TR * TC; i += 256) {
        const int r = i / TC, col = i - r * TC;
        const int iy = iy0 + r, ix = col - P;
        tile[i] = (iy >= 0 && iy < IH && ix >= 0 && ix < IW) ? xc[(int64_t)iy * IW + ix] : 0.0f;
    }
    __syncthreads();
    const float *__restrict__ wc = w + (int64_t)c * K * K;
    float wk[K * K];
#pragma unroll
    for (int i = 0; i < K * K; i++) wk[i] = wc[i];
    const float bc = b[c];
    float *__restrict__ oc = out + (int64_t)c * out_plane + (int64_t)oy0 * OW;
    for (int o = threadIdx.x; o < rows * OW; o += 256) {
        const int oy = o / OW, ox = o - oy * OW;
        const float *t = tile + oy * S * TC + ox * S;
        float v[K * K];
#pragma unroll
        for (int kh = 0; kh < K; kh++)
#pragma unroll
            for (int kw = 0; kw < K; kw++) v[kh * K + kw] = t[kh * TC + kw];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < K * K; i++) s = fmaf(v[i], wk[i], s);
        oc[o] = act_f(s + bc, act);
    }
}

// The same depthwise conv without LDS, for the stride-2 downsampling convs on
// large maps: a thread owns one output column of R consecutive output rows,
// loads the (R - 1) * S + K input rows x K columns those outputs read (clamped
// addresses, zero where the tap is padding) before the first FMA, and sums each
// output's taps in (kh, kw) order as k_dwconv does, so the results are
// bit-identical.  The LDS version stages a band with one load in flight per
// thread at a time; here every load of a thread is issued together.
template <int K, int S, int R>
__global__ __launch_bounds__(256) void k_dwconv_rows(const float *__restrict__ x, const float *__restrict__ w,
                                                     const float *__restrict__ b, float *__restrict__ out, int IH,
                                                     int IW, int OH, int OW, int P, int act, int groups,
                                                     int64_t in_plane, int64_t out_plane) {
    constexpr int TR = (R - 1) * S + K;
    const int c = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= groups * OW) return;
    const int g = i / OW, ox = i - g * OW;
    const int oy0 = g * R, iy0 = oy0 * S - P, ix0 = ox * S - P;
    const float *__restrict__ xc = x + (int64_t)c * in_plane;
    float v[TR][K];
#pragma unroll
    for (int r = 0; r < TR; r++) {
        const int iy = iy0 + r;
        const bool ry = iy >= 0 && iy < IH;
        const int64_t row = (int64_t)min(max(iy, 0), IH - 1) * IW;
#pragma unroll
        for (int kw = 0; kw < K; kw++) {
            const int ix = ix0 + kw;
            const float t = xc[row + min(max(ix, 0), IW - 1)];
            v[r][kw] = (ry && ix >= 0 && ix < IW) ? t : 0.0f;
        }
    }
    const float *__restrict__ wc = w + (int64_t)c * K * K;
    float wk[K * K];
#pragma unroll
    for (int j = 0; j < K * K; j++) wk[j] = wc[j];
    const float bc = b[c];
    float *__restrict__ oc = out + (int64_t)c * out_plane + ox;
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const int oy = oy0 + rr;
        float s = 0.0f;
#pragma unroll
        for (int kh = 0; kh < K; kh++)
#pragma unroll
            for (int kw = 0; kw < K; kw++) s = fmaf(v[rr * S + kh][kw], wk[kh * K + kw], s);
        if (oy < OH) oc[(int64_t)oy * OW] = act_f(s + bc, act);
    }
}

// 2x2 stride-1 max pool of x zero-padded by one column and one row at the
// right/bottom (ggml_pad + ggml_pool_2d, src/ppdoclayout.cpp:621-626): the
// output keeps x's size.
__global__ __launch_bounds__(256) void k_maxpool2_padend(const float *__restrict__ x, float *__restrict__ out,
                                                         int C, int H, int W) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)C * H * W) return;
    const int c = (int)(idx / ((int64_t)H * W));
    const int rem = (int)(idx - (int64_t)c * H * W);
    const int y = rem / W, xx = rem - y * W;
    const float *xc = x + (int64_t)c * H * W;
    const float v00 = xc[(int64_t)y * W + xx];
    const float v01 = xx + 1 < W ? xc[(int64_t)y * W + xx + 1] : 0.0f;
    const float v10 = y + 1 < H ? xc[(int64_t)(y + 1) * W + xx] : 0.0f;
    const float v11 = (xx + 1 < W && y + 1 < H) ? xc[(int64_t)(y + 1) * W + xx + 1] : 0.0f;
    out[idx] = fmaxf(fmaxf(v00, v01), fmaxf(v10, v11));
}

// The same pool, four outputs per thread (W % 4 == 0, 16-byte aligned planes:
// checked on the host): two aligned float4 row loads plus the next column of
// each row, one float4 store.  Same max order as k_maxpool2_padend.
__global__ __launch_bounds__(256) void k_maxpool2_padend4(const float *__restrict__ x, float *__restrict__ out,
                                                          int C, int H, int W) {
    const int W4 = W / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)C * H * W4) return;
    const int c = (int)(idx / ((int64_t)H * W4));
    const int rem = (int)(idx - (int64_t)c * H * W4);
    const int y = rem / W4, x0 = 4 * (rem - y * W4);
    const float *r0 = x + ((int64_t)c * H + y) * W + x0;
    const bool down = y + 1 < H, right = x0 + 4 < W;
    const float *r1 = down ? r0 + W : r0;
    const float4 a = *reinterpret_cast<const float4 *>(r0), b = *reinterpret_cast<const float4 *>(r1);
    const float a4 = right ? r0[4] : 0.0f, b4 = (right && down) ? r1[4] : 0.0f;
    const float bx = down ? b.x : 0.0f, by = down ? b.y : 0.0f, bz = down ? b.z : 0.0f, bw = down ? b.w : 0.0f;
    float4 o;
    o.x = fmaxf(fmaxf(a.x, a.y), fmaxf(bx, by));
    o.y = fmaxf(fmaxf(a.y, a.z), fmaxf(by, bz));
    o.z = fmaxf(fmaxf(a.z, a.w), fmaxf(bz, bw));
    o.w = fmaxf(fmaxf(a.w, a4), fmaxf(bw, b4));
    *reinterpret_cast<float4 *>(out + ((int64_t)c * H + y) * W + x0) = o;
}

// Interpolation (ggml_interpolate, src/ppdoclayout.cpp:670-672): nearest
// (src = floor(dst * in / out)) or bilinear with half-pixel centres and
// edge clamping; out = interp(x) + add (add may be null).
__device__ __forceinline__ float interp_at(const float *__restrict__ xc, int IH, int IW, int OH, int OW, int oy,
                                           int ox, int bilinear) {
    if (!bilinear) {
        const int iy = (int)((int64_t)oy * IH / OH), ix = (int)((int64_t)ox * IW / OW);
        return xc[(int64_t)iy * IW + ix];
    }
    const float sy = (float)OH / (float)IH, sx = (float)OW / (float)IW;
    const float fy = ((float)oy + 0.5f) / sy - 0.5f, fx = ((float)ox + 0.5f) / sx - 0.5f;
    const float fly = floorf(fy), flx = floorf(fx);
    int y0 = (int)fly, x0 = (int)flx;
    int y1 = y0 + 1, x1 = x0 + 1;
    y0 = max(0, min(y0, IH - 1));
    y1 = max(0, min(y1, IH - 1));
    x0 = max(0, min(x0, IW - 1));
    x1 = max(0, min(x1, IW - 1));
    const float dy = fmaxf(0.0f, fminf(fy - fly, 1.0f)), dx = fmaxf(0.0f, fminf(fx - flx, 1.0f));
    const float a = xc[(int64_t)y0 * IW + x0], bb = xc[(int64_t)y0 * IW + x1];
    const float cc = xc[(int64_t)y1 * IW + x0], d = xc[(int64_t)y1 * IW + x1];
    return a * (1.0f - dx) * (1.0f - dy) + bb * dx * (1.0f - dy) + cc * (1.0f - dx) * dy + d * dx * dy;
}

__global__ __launch_bounds__(256) void k_interp(const float *__restrict__ x, const float *__restrict__ add,
                                                float *__restrict__ out, int C, int IH, int IW, int OH, int OW,
                                                int bilinear) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)C * OH * OW) return;
    const int c = (int)(idx / ((int64_t)OH * OW));
    const int rem = (int)(idx - (int64_t)c * OH * OW);
    const int oy = rem / OW, ox = rem - oy * OW;
    float v = interp_at(x + (int64_t)c * IH * IW, IH, IW, OH, OW, oy, ox, bilinear);
    if (add) v += add[idx];
    out[idx] = v;
}

// Four consecutive outputs per thread (OW % 4 == 0, 16-byte aligned out /
// add: checked on the host), one float4 store; same values as k_interp.
__global__ __launch_bounds__(256) void k_interp4(const float *__restrict__ x, const float *__restrict__ add,
                                                 float *__restrict__ out, int C, int IH, int IW, int OH, int OW,
                                                 int bilinear) {
    const int OW4 = OW / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)C * OH * OW4) return;
    const int c = (int)(idx / ((int64_t)OH * OW4));
    const int rem = (int)(idx - (int64_t)c * OH * OW4);
    const int oy = rem / OW4, ox = 4 * (rem - oy * OW4);
    const float *xc = x + (int64_t)c * IH * IW;
    float4 v = make_float4(interp_at(xc, IH, IW, OH, OW, oy, ox, bilinear),
                           interp_at(xc, IH, IW, OH, OW, oy, ox + 1, bilinear),
                           interp_at(xc, IH, IW, OH, OW, oy, ox + 2, bilinear),
                           interp_at(xc, IH, IW, OH, OW, oy, ox + 3, bilinear));
    const int64_t o = ((int64_t)c * OH + oy) * OW + ox;
    if (add) {
        const float4 a = *reinterpret_cast<const float4 *>(add + o);
        v.x += a.x;
        v.y += a.y;
        v.z += a.z;
        v.w += a.w;
    }
    *reinterpret_cast<float4 *>(out + o) = v;
}

// Exact 2x upsampling (OH = 2 IH, OW = 2 IW, OW % 4 == 0, 16-byte aligned out
// and add), four outputs of one row per thread.  Nearest: input column ox / 2.
// Bilinear: the scale is the constant 2, so the source coordinates are
// (o + 0.5) / 2 - 0.5 exactly as in interp_at, and the four outputs
// 4j .. 4j+3 read input columns 2j-1 .. 2j+2 (clamped) of two rows, loaded
// once; each output is formed by interp_at's expression in its order, so the
// values are bit-identical to k_interp4.  32-bit index math (the host checks
// the extent).
template <int BIL>
__global__ __launch_bounds__(256) void k_up2x4(const float *__restrict__ x, const float *__restrict__ add,
                                               float *__restrict__ out, int C, int IH, int IW) {
    const int OH = 2 * IH, OW = 2 * IW, OW4 = OW / 4;
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint32_t)C * (uint32_t)(OH * OW4)) return;
    const uint32_t per = (uint32_t)(OH * OW4);
    const uint32_t c = idx / per, rem = idx - c * per;
    const int oy = (int)(rem / (uint32_t)OW4), j = (int)(rem - (uint32_t)oy * OW4), ox = 4 * j;
    const float *__restrict__ xc = x + c * (uint32_t)(IH * IW);
    float v[4];
    if (!BIL) {
        const float *r = xc + (oy >> 1) * IW + 2 * j;
        const float a = r[0], b = r[1];
        v[0] = a, v[1] = a, v[2] = b, v[3] = b;
    } else {
        const float fy = ((float)oy + 0.5f) / 2.0f - 0.5f;
        const float fly = floorf(fy);
        const int y0 = max(0, min((int)fly, IH - 1)), y1 = max(0, min((int)fly + 1, IH - 1));
        const float dy = fmaxf(0.0f, fminf(fy - fly, 1.0f));
        float r0[4], r1[4];  // columns 2j-1 .. 2j+2, clamped
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int cx = max(0, min(2 * j - 1 + e, IW - 1));
            r0[e] = xc[y0 * IW + cx];
            r1[e] = xc[y1 * IW + cx];
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float fx = ((float)(ox + e) + 0.5f) / 2.0f - 0.5f;
            const float flx = floorf(fx);
            const float dx = fmaxf(0.0f, fminf(fx - flx, 1.0f));
            const int l = (int)flx - (2 * j - 1);  // 0 or 1 or 2: the left column within r0 / r1
            const float a = r0[l], bb = r0[l + 1], cc = r1[l], d = r1[l + 1];
            v[e] = a * (1.0f - dx) * (1.0f - dy) + bb * dx * (1.0f - dy) + cc * (1.0f - dx) * dy + d * dx * dy;
        }
    }
    const uint32_t o = (c * (uint32_t)OH + (uint32_t)oy) * (uint32_t)OW + (uint32_t)ox;
    if (add) {
        const float4 a = *reinterpret_cast<const float4 *>(add + o);
        v[0] += a.x;
        v[1] += a.y;
        v[2] += a.z;
        v[3] += a.w;
    }
    *reinterpret_cast<float4 *>(out + o) = make_float4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------------------
// Layer norm over the 256 features of each token (ggml_norm eps 1e-5, then
// * gamma + beta, src/ppdoclayout.cpp:550-554), with the residual sum of
// the reference's ln(x + y) fused: out = LN(a + b).  One wave per token,
// 4 features per lane; mean and variance by wave reductions.  out_chw
// stores the result channel-major ([256][T]) instead of token-major.
__global__ __launch_bounds__(256) void k_layernorm(const float *__restrict__ a, const float *__restrict__ b,
                                                   const float *__restrict__ gamma,
                                                   const float *__restrict__ beta, float *__restrict__ out,
                                                   int T, float eps, int out_chw, const float *__restrict__ row_mask,
                                                   const float *__restrict__ row_fill) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const float4 av = *reinterpret_cast<const float4 *>(a + (int64_t)t * kDM + lane * 4);
    // without b the second row load re-reads a (selected address, no branch
    // between the loads) and is not added
    const float4 bv0 = *reinterpret_cast<const float4 *>((b ? b : a) + (int64_t)t * kDM + lane * 4);
    const float4 gv = *reinterpret_cast<const float4 *>(gamma + lane * 4);
    const float4 bv = *reinterpret_cast<const float4 *>(beta + lane * 4);
    // masked rows (row_mask[t] == 0) take row_fill instead of a's row
    const float4 fv = *reinterpret_cast<const float4 *>((row_mask ? row_fill : a) + lane * 4);
    const bool fill = row_mask && row_mask[t] == 0.0f;
    __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the reductions
    float v[4] = {fill ? fv.x : av.x, fill ? fv.y : av.y, fill ? fv.z : av.z, fill ? fv.w : av.w};
    if (b) {
        v[0] += bv0.x;
        v[1] += bv0.y;
        v[2] += bv0.z;
        v[3] += bv0.w;
    }
    const float mean = wave_sum((v[0] + v[1]) + (v[2] + v[3])) / (float)kDM;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] -= mean;
        q += v[i] * v[i];
    }
    const float scale = 1.0f / sqrtf(wave_sum(q) / (float)kDM + eps);
    const float y[4] = {v[0] * scale * gv.x + bv.x, v[1] * scale * gv.y + bv.y, v[2] * scale * gv.z + bv.z,
                        v[3] * scale * gv.w + bv.w};
    if (out_chw) {
#pragma unroll
        for (int i = 0; i < 4; i++) out[(int64_t)(lane * 4 + i) * T + t] = y[i];
    } else {
        *reinterpret_cast<float4 *>(out + (int64_t)t * kDM + lane * 4) = make_float4(y[0], y[1], y[2], y[3]);
    }
}

// ---------------------------------------------------------------------------
// Multi-head attention core (src/ppdoclayout.cpp:572-587): per head h,
// out[t][h*32+c] = sum_s softmax_s(q_t . k_s / sqrt(32)) v[s][h*32+c].
// q, k, v are token-major with row strides ldq/ldk/ldv.
//
// On the FP32 matrix cores (v_mfma_f32_32x32x2_f32).  A block owns one head
// and 32 queries; its 8 waves take interleaved 32-key chunks and keep an
// online softmax each, merged at the end (the merge buffers reuse the K/V
// staging space once every wave is done with it).  Per chunk a wave computes the
// transposed scores S^T = K Q^T (32 keys x 32 queries), so each lane's
// accumulator column is one query: the row max / sum over keys stay within a
// lane pair, and the accumulator registers of S^T are directly the B operand
// of O^T += V^T P^T (register r holds keys 8(r/4) + r%4 in lanes 0-31 and 4
// more in lanes 32-63, which fixes the key each lane supplies on the A side).
// K and V chunks pass through a per-wave LDS slice; a wave issues the loads
// of all its chunks (at most kAttCPW) before the first one's math.  The
// block's Q goes through LDS once; after that barrier, none until the merge.
typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr int kAttQ = 32, kAttWaves = 8, kAttThreads = 64 * kAttWaves;
constexpr int kAttCPW = 3;  // key chunks per wave held in registers: T <= 8 * 3 * 32 = 768

__global__ __launch_bounds__(kAttThreads) void k_attention(const float *__restrict__ q, int ldq,
                                                           const float *__restrict__ k, int ldk,
                                                           const float *__restrict__ v, int ldv,
                                                           float *__restrict__ out, int ldo, int T, float scale) {
    __shared__ float stage[2][kAttWaves][32][kHD + 1];  // K and V chunks per wave; then the merge tiles
    __shared__ float mw[kAttWaves][kAttQ], lw[kAttWaves][kAttQ];
    float (*Ks)[32][kHD + 1] = stage[0];
    float (*Vs)[32][kHD + 1] = stage[1];
    float (*ow)[kHD][kAttQ + 1] = stage[0];  // [wave][d][q], valid after the loop barrier
    const int h = blockIdx.y, q0 = blockIdx.x * kAttQ;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l32 = lane & 31, hi = lane >> 5;

    // This wave's K/V chunks (c = wave, wave + 8, ...; at most kAttCPW), all
    // of their loads issued before any math: lane = key row lane/2, 16
    // consecutive channels (lane%2)*16; rows past T read row T - 1 and are
    // zeroed when staged.
    const int row = lane >> 1, c0 = (lane & 1) * 16;
    float4 kv[kAttCPW][8];
#pragma unroll
    for (int u = 0; u < kAttCPW; u++) {
        const int s_ = min((wave + kAttWaves * u) * 32 + row, T - 1);
        const float4 *kr = reinterpret_cast<const float4 *>(k + (int64_t)s_ * ldk + h * kHD + c0);
        const float4 *vr = reinterpret_cast<const float4 *>(v + (int64_t)s_ * ldv + h * kHD + c0);
#pragma unroll
        for (int j = 0; j < 4; j++) kv[u][j] = kr[j], kv[u][4 + j] = vr[j];
    }
    // Q of the block's 32 queries through LDS (one float4 per thread of
    // the first four waves), read back as the B operand of S^T: Q^T[d][q],
    // lane supplies d = 2*st + hi of query l32
    __shared__ float qs[kAttQ][kHD + 1];
    if (threadIdx.x < kAttQ * kHD / 4) {
        const int qi = threadIdx.x >> 3, d4 = (threadIdx.x & 7) * 4;
        const float4 qv =
            *reinterpret_cast<const float4 *>(q + (int64_t)min(q0 + qi, T - 1) * ldq + h * kHD + d4);
        const bool in = q0 + qi < T;
        qs[qi][d4 + 0] = in ? qv.x : 0.0f;
        qs[qi][d4 + 1] = in ? qv.y : 0.0f;
        qs[qi][d4 + 2] = in ? qv.z : 0.0f;
        qs[qi][d4 + 3] = in ? qv.w : 0.0f;
    }
    __syncthreads();
    float qf[kHD / 2];
#pragma unroll
    for (int st = 0; st < kHD / 2; st++) qf[st] = qs[l32][2 * st + hi];
    f32x16_t o;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;

#pragma unroll
    for (int u = 0; u < kAttCPW; u++) {
        const int c = wave + kAttWaves * u;
        if (c * 32 >= T) break;  // wave-uniform
        const int key0 = c * 32;
        {
            const bool in = key0 + row < T;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 a = kv[u][j], b = kv[u][4 + j];
                Ks[wave][row][c0 + 4 * j + 0] = in ? a.x : 0.0f;
                Ks[wave][row][c0 + 4 * j + 1] = in ? a.y : 0.0f;
                Ks[wave][row][c0 + 4 * j + 2] = in ? a.z : 0.0f;
                Ks[wave][row][c0 + 4 * j + 3] = in ? a.w : 0.0f;
                Vs[wave][row][c0 + 4 * j + 0] = in ? b.x : 0.0f;
                Vs[wave][row][c0 + 4 * j + 1] = in ? b.y : 0.0f;
                Vs[wave][row][c0 + 4 * j + 2] = in ? b.z : 0.0f;
                Vs[wave][row][c0 + 4 * j + 3] = in ? b.w : 0.0f;
            }
        }
        __builtin_amdgcn_wave_barrier();
        // S^T[key][q]: A = K (lane: key l32, d = 2st + hi)
        f32x16_t sc;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < kHD / 2; st++)
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[wave][l32][2 * st + hi], qf[st], sc, 0, 0, 0);
        // scale, mask keys past T, chunk max per query (lane pair l32, l32 + 32)
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = key0 + 8 * (r >> 2) + 4 * hi + (r & 3);
            sc[r] = key < T ? sc[r] * scale : -INFINITY;
            mx = fmaxf(mx, sc[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);  // finite: the chunk holds at least one key < T
        const float corr = expf(m - mn);
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            sc[r] = expf(sc[r] - mn);
            ps += sc[r];
        }
        ps += __shfl_xor(ps, 32);
        lsum = lsum * corr + ps;
        m = mn;
#pragma unroll
        for (int r = 0; r < 16; r++) o[r] *= corr;
        // O^T[d][q] += V^T P^T: step st pairs keys 8(st/4) + st%4 (+4 in the upper half)
#pragma unroll
        for (int st = 0; st < 16; st++)
            o = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[wave][8 * (st >> 2) + 4 * hi + (st & 3)][l32], sc[st], o, 0,
                                                     0, 0);
        __builtin_amdgcn_wave_barrier();
    }

    // merge the waves' partial softmaxes
    __syncthreads();  // every wave is done with its K/V slice (ow aliases it)
    if (hi == 0) {
        mw[wave][l32] = m;
        lw[wave][l32] = lsum;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) ow[wave][8 * (r >> 2) + 4 * hi + (r & 3)][l32] = o[r];
    __syncthreads();
    const int d = threadIdx.x & 31;
#pragma unroll
    for (int j = 0; j < kAttQ * 32 / kAttThreads; j++) {
        const int qi = (threadIdx.x >> 5) + (kAttThreads / 32) * j, t = q0 + qi;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kAttWaves; w++) M = fmaxf(M, mw[w][qi]);
        float L = 0.0f, acc = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttWaves; w++) {
            const float e = mw[w][qi] == -INFINITY ? 0.0f : expf(mw[w][qi] - M);
            L += e * lw[w][qi];
            acc += e * ow[w][d][qi];
        }
        if (t < T) out[(int64_t)t * ldo + h * kHD + d] = acc / L;
    }
}

// The same attention with 16 queries per block on v_mfma_f32_16x16x4f32: twice
// the blocks (152 for 300 tokens) and half the dependent MFMA chain per key
// chunk.  Per 32-key chunk a wave computes two 16-key tiles of S^T = K Q^T
// (lane l: query l%16, keys 4(l/16) + r of register r), and those registers
// are the B operand of O^T += V^T P^T directly: step (tile t, register r)
// contracts keys 16t + 4g + r, g = lane group, and the A operand reads V at
// the same keys.  Loads, masking, the online softmax and the merge follow
// k_attention.
constexpr int kA16Q = 16;
typedef float f32x4_att __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kAttThreads) void k_attention16(const float *__restrict__ q, int ldq,
                                                             const float *__restrict__ k, int ldk,
                                                             const float *__restrict__ v, int ldv,
                                                             float *__restrict__ out, int ldo, int T, float scale) {
    __shared__ float stage[2][kAttWaves][32][kHD + 1];  // K and V chunks per wave; then the merge tiles
    __shared__ float mw[kAttWaves][kA16Q], lw[kAttWaves][kA16Q];
    __shared__ float qs[kA16Q][kHD + 1];
    float (*Ks)[32][kHD + 1] = stage[0];
    float (*Vs)[32][kHD + 1] = stage[1];
    float (*ow)[kHD][kA16Q + 1] = reinterpret_cast<float (*)[kHD][kA16Q + 1]>(&stage[0][0][0][0]);
    const int h = blockIdx.y, q0 = blockIdx.x * kA16Q;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c16 = lane & 15, g = lane >> 4;

    const int row = lane >> 1, c0 = (lane & 1) * 16;
    float4 kv[kAttCPW][8];
#pragma unroll
    for (int u = 0; u < kAttCPW; u++) {
        const int s_ = min((wave + kAttWaves * u) * 32 + row, T - 1);
        const float4 *kr = reinterpret_cast<const float4 *>(k + (int64_t)s_ * ldk + h * kHD + c0);
        const float4 *vr = reinterpret_cast<const float4 *>(v + (int64_t)s_ * ldv + h * kHD + c0);
#pragma unroll
        for (int j = 0; j < 4; j++) kv[u][j] = kr[j], kv[u][4 + j] = vr[j];
    }
    if (threadIdx.x < kA16Q * kHD / 4) {
        const int qi = threadIdx.x >> 3, d4 = (threadIdx.x & 7) * 4;
        const float4 qv =
            *reinterpret_cast<const float4 *>(q + (int64_t)min(q0 + qi, T - 1) * ldq + h * kHD + d4);
        const bool in = q0 + qi < T;
        qs[qi][d4 + 0] = in ? qv.x : 0.0f;
        qs[qi][d4 + 1] = in ? qv.y : 0.0f;
        qs[qi][d4 + 2] = in ? qv.z : 0.0f;
        qs[qi][d4 + 3] = in ? qv.w : 0.0f;
    }
    __syncthreads();
    // B operand of S^T: Q^T[d][q], lane supplies d = 4 st + g of query c16
    float qf[kHD / 4];
#pragma unroll
    for (int st = 0; st < kHD / 4; st++) qf[st] = qs[c16][4 * st + g];
    f32x4_att o[2];
#pragma unroll
    for (int t = 0; t < 2; t++) o[t] = f32x4_att{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, lsum = 0.0f;

#pragma unroll
    for (int u = 0; u < kAttCPW; u++) {
        const int c = wave + kAttWaves * u;
        if (c * 32 >= T) break;  // wave-uniform
        const int key0 = c * 32;
        {
            const bool in = key0 + row < T;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 a = kv[u][j], b = kv[u][4 + j];
                Ks[wave][row][c0 + 4 * j + 0] = in ? a.x : 0.0f;
                Ks[wave][row][c0 + 4 * j + 1] = in ? a.y : 0.0f;
                Ks[wave][row][c0 + 4 * j + 2] = in ? a.z : 0.0f;
                Ks[wave][row][c0 + 4 * j + 3] = in ? a.w : 0.0f;
                Vs[wave][row][c0 + 4 * j + 0] = in ? b.x : 0.0f;
                Vs[wave][row][c0 + 4 * j + 1] = in ? b.y : 0.0f;
                Vs[wave][row][c0 + 4 * j + 2] = in ? b.z : 0.0f;
                Vs[wave][row][c0 + 4 * j + 3] = in ? b.w : 0.0f;
            }
        }
        __builtin_amdgcn_wave_barrier();
        // S^T tiles: A = K (lane: key 16 t + c16, d = 4 st + g)
        f32x4_att sc[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            sc[t] = f32x4_att{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < kHD / 4; st++)
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(Ks[wave][16 * t + c16][4 * st + g], qf[st], sc[t], 0, 0,
                                                             0);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = key0 + 16 * t + 4 * g + r;
                sc[t][r] = key < T ? sc[t][r] * scale : -INFINITY;
                mx = fmaxf(mx, sc[t][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);  // finite: the chunk holds at least one key < T
        const float corr = expf(m - mn);
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sc[t][r] = expf(sc[t][r] - mn);
                ps += sc[t][r];
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        lsum = lsum * corr + ps;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) o[dt][r] *= corr;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(Vs[wave][16 * t + 4 * g + r][16 * dt + c16], sc[t][r],
                                                                 o[dt], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
    }

    __syncthreads();  // every wave is done with its K/V slice (ow aliases it)
    if (g == 0) {
        mw[wave][c16] = m;
        lw[wave][c16] = lsum;
    }
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++) ow[wave][16 * dt + 4 * g + r][c16] = o[dt][r];
    __syncthreads();
    const int d = threadIdx.x & 31, qi = threadIdx.x >> 5, t = q0 + qi;  // 16 queries x 32 d = 512 threads
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttWaves; w++) M = fmaxf(M, mw[w][qi]);
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttWaves; w++) {
        const float e = mw[w][qi] == -INFINITY ? 0.0f : expf(mw[w][qi] - M);
        L += e * lw[w][qi];
        acc += e * ow[w][d][qi];
    }
    if (t < T) out[(int64_t)t * ldo + h * kHD + d] = acc / L;
}

// ---------------------------------------------------------------------------
// Elementwise helpers.
__global__ __launch_bounds__(256) void k_add(const float *__restrict__ a, const float *__restrict__ b,
                                             float *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// out[t][c] = x[t][c] * mask[t]  (memory = source * valid, src/ppdoclayout.cpp:801)
__global__ __launch_bounds__(256) void k_mul_rows(const float *__restrict__ x, const float *__restrict__ mask,
                                                  float *__restrict__ out, int64_t T, int D) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < T * D) out[i] = x[i] * mask[i / D];
}

// Box refinement (src/ppdoclayout.cpp:860-862): ref = sigmoid(delta + inv_sigmoid(ref)).
// With delta == null: ref = sigmoid(ref) (the initial reference).
__global__ __launch_bounds__(256) void k_box_update(const float *__restrict__ delta, float *__restrict__ ref,
                                                    int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    ref[i] = delta ? refine_box(delta[i], ref[i]) : 1.0f / (1.0f + expf(-ref[i]));
}

// target = om[idx]: ggml_get_rows of 256-wide token rows (src/ppdoclayout.cpp:805)
__global__ __launch_bounds__(256) void k_get_rows(const float *__restrict__ src, const int32_t *__restrict__ idx,
                                                  float *__restrict__ out, int nrows) {
    const int r = blockIdx.x, c = threadIdx.x;
    if (r >= nrows) return;
    out[(int64_t)r * kDM + c] = src[(int64_t)idx[r] * kDM + c];
}

// Reading-order logits (src/ppdoclayout.cpp:874-876):
// order[m + NQ*n] = scale * sum_c gp[m][64 + c] * gp[n][c]  (ggml_mul_mat(kv, qv))
__global__ __launch_bounds__(256) void k_order(const float *__restrict__ gp, float *__restrict__ out, int nq,
                                               int hd, float scale) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)nq * nq) return;
    const int m = (int)(i % nq), n = (int)(i / nq);
    const float *kv = gp + (int64_t)m * 2 * hd + hd, *qv = gp + (int64_t)n * 2 * hd;
    // float4 loads and four interleaved partial sums (hd % 4 == 0, 16-byte
    // aligned rows: checked on the host); partials added in a fixed order
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    for (int c = 0; c < hd; c += 4) {
        const float4 a = *reinterpret_cast<const float4 *>(kv + c), b = *reinterpret_cast<const float4 *>(qv + c);
        s0 = fmaf(a.x, b.x, s0);
        s1 = fmaf(a.y, b.y, s1);
        s2 = fmaf(a.z, b.z, s2);
        s3 = fmaf(a.w, b.w, s3);
    }
    out[i] = ((s0 + s1) + (s2 + s3)) * scale;
}

// CHW [C][P] -> token-major [P][C] (the reference's to_seq / cont(permute)),
// through a 32x32 LDS tile.
__global__ __launch_bounds__(256) void k_transpose(const float *__restrict__ in, float *__restrict__ out,
                                                   int rows, int cols, int ldo) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8)
        if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = in[(int64_t)(r0 + r) * cols + c0 + tx];
    __syncthreads();
    for (int c = ty; c < 32; c += 8)
        if (c0 + c < cols && r0 + tx < rows) out[(int64_t)(c0 + c) * ldo + r0 + tx] = tile[tx][c];
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t dwconv(const float *x, const float *w, const float *b, float *out, int C, int IH, int IW, int K, int S,
                  int P, int act, int64_t in_plane, int64_t out_plane, hipStream_t s) {
    const int OH = (IH + 2 * P - K) / S + 1, OW = (IW + 2 * P - K) / S + 1;
    const int TC = IW + 2 * P;
    // the band's staged rows must fit the LDS tile: (RB - 1) * S + K rows of TC
    const int max_rows = kDwLds / TC;
    if (C < 1 || OH < 1 || OW < 1 || C > 65535 || max_rows < K || (K != 3 && K != 5) ||
        in_plane < (int64_t)IH * IW || out_plane < (int64_t)OH * OW)
        return hipErrorInvalidValue;
    // stride 2 (the stage downsampling convs): the register version
    // (PPDL_DW_ROWS=0 keeps the LDS one).  Graph A/B: -3 us per replay over
    // the three downsampling convs.  With stride 1 (the 5x5 convs on the
    // 50x50 and 25x25 maps, 2 rows per thread) it was 90 us slower: the LDS
    // band there is read 25 times per element.
    const char *er = getenv("PPDL_DW_ROWS");
    if (K == 3 && S == 2 && !(er && er[0] == '0')) {
        constexpr int R = 4;
        const int groups = (OH + R - 1) / R;
        const dim3 g2((unsigned)(((int64_t)groups * OW + 255) / 256), C);
        hipLaunchKernelGGL((k_dwconv_rows<3, 2, R>), g2, dim3(256), 0, s, x, w, b, out, IH, IW, OH, OW, P, act,
                           groups, in_plane, out_plane);
        return hipGetLastError();
    }
    const int bands = std::max(1, (2048 + C - 1) / C);
    const int RB = std::max(1, std::min((OH + bands - 1) / bands, (max_rows - K) / S + 1));
    const dim3 grid((OH + RB - 1) / RB, C);
    if (K == 3)
        hipLaunchKernelGGL(k_dwconv<3>, grid, dim3(256), 0, s, x, w, b, out, C, IH, IW, OH, OW, S, P, act, RB,
                           in_plane, out_plane);
    else
        hipLaunchKernelGGL(k_dwconv<5>, grid, dim3(256), 0, s, x, w, b, out, C, IH, IW, OH, OW, S, P, act, RB,
                           in_plane, out_plane);
    return hipGetLastError();
}

hipError_t maxpool2_padend(const float *x, float *out, int C, int H, int W, hipStream_t s) {
    if (W % 4 == 0 && (((uintptr_t)x | (uintptr_t)out) & 15) == 0)
        hipLaunchKernelGGL(k_maxpool2_padend4, dim3(blocks_for((int64_t)C * H * (W / 4))), dim3(256), 0, s, x, out, C,
                           H, W);
    else
        hipLaunchKernelGGL(k_maxpool2_padend, dim3(blocks_for((int64_t)C * H * W)), dim3(256), 0, s, x, out, C, H, W);
    return hipGetLastError();
}

hipError_t interp(const float *x, const float *add, float *out, int C, int IH, int IW, int OH, int OW,
                  int bilinear, hipStream_t s) {
    const char *eu = getenv("PPDL_UP2X");
    if (!(eu && eu[0] == '0') && OH == 2 * IH && OW == 2 * IW && OW % 4 == 0 &&
        (int64_t)C * OH * OW < (1LL << 31) && (((uintptr_t)out | (uintptr_t)add) & 15) == 0) {
        const unsigned blocks = blocks_for((int64_t)C * OH * (OW / 4));
        if (bilinear)
            hipLaunchKernelGGL(k_up2x4<1>, dim3(blocks), dim3(256), 0, s, x, add, out, C, IH, IW);
        else
            hipLaunchKernelGGL(k_up2x4<0>, dim3(blocks), dim3(256), 0, s, x, add, out, C, IH, IW);
        return hipGetLastError();
    }
    if (OW % 4 == 0 && (((uintptr_t)out | (uintptr_t)add) & 15) == 0) {
        hipLaunchKernelGGL(k_interp4, dim3(blocks_for((int64_t)C * OH * (OW / 4))), dim3(256), 0, s, x, add, out, C,
                           IH, IW, OH, OW, bilinear);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_interp, dim3(blocks_for((int64_t)C * OH * OW)), dim3(256), 0, s, x, add, out, C, IH, IW,
                       OH, OW, bilinear);
    return hipGetLastError();
}

// One lane stores the device's constant-rate wall clock (profiling only; a
// vector store from a register).
__global__ void k_stamp(unsigned long long *slot) {
    if (threadIdx.x == 0) *slot = wall_clock64();
}

hipError_t stamp(unsigned long long *slot, hipStream_t s) {
    hipLaunchKernelGGL(k_stamp, dim3(1), dim3(64), 0, s, slot);
    return hipGetLastError();
}

hipError_t layernorm(const float *a, const float *b, const float *gamma, const float *beta, float *out, int T,
                     int out_chw, hipStream_t s, const float *row_mask, const float *row_fill) {
    // rows, gamma, beta, the fill row and (token-major) out are accessed as float4
    if ((((uintptr_t)a | (uintptr_t)b | (uintptr_t)gamma | (uintptr_t)beta | (uintptr_t)out |
          (uintptr_t)row_fill) & 15) != 0 || (row_mask && !row_fill) || (row_mask && b))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_layernorm, dim3((T + 3) / 4), dim3(256), 0, s, a, b, gamma, beta, out, T, 1e-5f, out_chw,
                       row_mask, row_fill);
    return hipGetLastError();
}

hipError_t attention(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv, float *out,
                     int ldo, int T, hipStream_t s) {
    // K, V and Q rows are read as float4; every key chunk fits the waves' registers
    if (T < 1 || T > kAttWaves * kAttCPW * 32 || ldk % 4 || ldv % 4 || ldq % 4 ||
        (((uintptr_t)k | (uintptr_t)v | (uintptr_t)q) & 15))
        return hipErrorInvalidValue;
    // 16 queries per block for the decoder's 300 tokens (PPDL_ATT16=0: never);
    // with 625 tokens (AIFI) the 32-query kernel is faster in the graph
    // (15.4 against 18.9 us: each wave already holds 3 key chunks)
    const char *e16 = getenv("PPDL_ATT16");
    if (!(e16 && e16[0] == '0') && T <= 320)
        hipLaunchKernelGGL(k_attention16, dim3((T + kA16Q - 1) / kA16Q, kNH), dim3(kAttThreads), 0, s, q, ldq, k, ldk,
                           v, ldv, out, ldo, T, 1.0f / sqrtf((float)kHD));
    else
        hipLaunchKernelGGL(k_attention, dim3((T + kAttQ - 1) / kAttQ, kNH), dim3(kAttThreads), 0, s, q, ldq, k, ldk,
                           v, ldv, out, ldo, T, 1.0f / sqrtf((float)kHD));
    return hipGetLastError();
}

hipError_t add(const float *a, const float *b, float *out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_add, dim3(blocks_for(n)), dim3(256), 0, s, a, b, out, n);
    return hipGetLastError();
}

hipError_t mul_rows(const float *x, const float *mask, float *out, int64_t T, int D, hipStream_t s) {
    hipLaunchKernelGGL(k_mul_rows, dim3(blocks_for(T * D)), dim3(256), 0, s, x, mask, out, T, D);
    return hipGetLastError();
}

hipError_t box_update(const float *delta, float *ref, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_box_update, dim3(blocks_for(n)), dim3(256), 0, s, delta, ref, n);
    return hipGetLastError();
}

hipError_t get_rows(const float *src, const int32_t *idx, float *out, int nrows, hipStream_t s) {
    hipLaunchKernelGGL(k_get_rows, dim3(nrows), dim3(kDM), 0, s, src, idx, out, nrows);
    return hipGetLastError();
}

hipError_t order_logits(const float *gp, float *out, int nq, int hd, float scale, hipStream_t s) {
    if (hd % 4 != 0 || (((uintptr_t)gp) & 15) != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_order, dim3(blocks_for((int64_t)nq * nq)), dim3(256), 0, s, gp, out, nq, hd, scale);
    return hipGetLastError();
}

hipError_t transpose(const float *in, float *out, int rows, int cols, int ldo, hipStream_t s) {
    hipLaunchKernelGGL(k_transpose, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(256), 0, s, in, out, rows, cols,
                       ldo);
    return hipGetLastError();
}

}  // namespace ppdl
