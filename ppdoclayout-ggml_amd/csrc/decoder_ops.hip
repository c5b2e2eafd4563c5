// Decoder-side tagged ops: MSDeformAttn sampling (op 2), mask -> box (op 1)
// and top-300 query selection (op 13).
//
// Semantics follow the reference's CPU ops, which define the results:
// op_msdeform (src/ppdoclayout.cpp:148-198), op_mask_box (:100-140),
// op_topk300 (:75-96).  Float contraction is off in this file so every
// multiply and add rounds where the CPU op's source rounds, except the
// explicit fmaf of the sampling accumulation (one fused multiply-add per
// corner tap, the reference GPU kernel's numerical contract).
#include "ppdl_internal.h"

#pragma clang fp contract(off)

namespace ppdl {
namespace {

// ---------------------------------------------------------------------------
// MSDeformAttn: one 256-thread block per query; wave w serves heads 2w, 2w+1
// (lane>>5 picks the head, lane&31 the channel).  For a fixed (head, point,
// corner) the 32 lanes of a head read 32 consecutive floats of the value map,
// so every gather is one 128-byte segment.
//   val  (13125, 256) token-major       off (NQ, 192) [((h*3+l)*4+p)*2+xy]
//   awr  (NQ, 96) pre-softmax [h*12 + l*4 + p]   ref (NQ, 4) cxcywh
// val, off and awr rows may be strided (ldv, ldo, ldw floats): slices of a
// wider projection.
//
// The sampling arithmetic is the same for the 32 lanes of a head, so it is
// done once per sample: lane j < 12 of a head owns sample j = l*4 + p (its
// logit, its offset pair, its 4 corners) and publishes the corners' tokens
// and weights in LDS; then every lane reads its head's 48 (token, weight)
// pairs as broadcasts, issues the 48 gathers together and accumulates in
// the reference's l -> p -> corner order.  The softmax max is a shuffle
// reduction (exact in any order); its sum adds the 12 terms in index order,
// as the reference does.
struct MsCorner {
    int tok;   // -1: the corner is skipped
    float wv;  // attention weight x bilinear weight
};

__global__ __launch_bounds__(256) void k_msdeform(const float *__restrict__ val,
                                                  const float *__restrict__ off,
                                                  const float *__restrict__ awr,
                                                  const float *__restrict__ ref,
                                                  float *__restrict__ out, int nq, int ldv, int ldo,
                                                  int ldw) {
    constexpr int kS = 3 * 4 * 4;
    __shared__ __attribute__((aligned(16))) MsCorner corners[8][kS];
    const int q = blockIdx.x;
    if (q >= nq) return;  // the whole block, before any barrier
    const int h = threadIdx.x >> 5, c = threadIdx.x & 31;
    const int j = min(c, 11);  // this lane's sample (lanes 12-31 shadow sample 11)

    const float a = awr[(int64_t)q * ldw + h * 12 + j];
    float amax = c < 12 ? a : -INFINITY;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float e = expf(a - amax);
    float wsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 12; i++) wsum += __shfl(e, i, 32);  // lane i of this head's 32
    const float wt = e / wsum;

    if (c < 12) {
        const int l = j >> 2;
        const int W = l == 0 ? 100 : l == 1 ? 50 : 25, H = W;
        const int st = l == 0 ? 0 : l == 1 ? 10000 : 12500;
        const float rx = ref[q * 4 + 0], ry = ref[q * 4 + 1];
        const float rw = ref[q * 4 + 2], rh = ref[q * 4 + 3];
        const float *o = off + (int64_t)q * ldo + h * 24 + j * 2;
        const float lx = rx + o[0] / 4.0f * rw * 0.5f;
        const float ly = ry + o[1] / 4.0f * rh * 0.5f;
        // grid_sample bilinear, zero padding, align_corners = false.  The
        // clamp only keeps the float->int conversion defined: any sample
        // beyond it has both corner columns (rows) outside the map.
        const float fx = fminf(fmaxf(lx * (float)W - 0.5f, -2.0f), (float)W + 1.0f);
        const float fy = fminf(fmaxf(ly * (float)H - 0.5f, -2.0f), (float)H + 1.0f);
        const int x0 = (int)floorf(fx), y0 = (int)floorf(fy);
        const float tx = fx - (float)x0, ty = fy - (float)y0;
        const float cw[4] = {(1.0f - tx) * (1.0f - ty), tx * (1.0f - ty), (1.0f - tx) * ty, tx * ty};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // a corner outside the map or with zero bilinear weight is
            // skipped, as the reference skips it
            const int xx = x0 + (k & 1), yy = y0 + (k >> 1);
            const bool in = xx >= 0 && xx < W && yy >= 0 && yy < H && cw[k] != 0.0f;
            corners[h][j * 4 + k] = MsCorner{in ? st + yy * W + xx : -1, wt * cw[k]};
        }
    }
    __syncthreads();

    // A skipped corner's gather reads token 0 (any valid address) and a
    // select, not a multiply by zero, leaves the sum as it was, so a
    // non-finite value there cannot reach the output.
    const float *vh = val + h * kHD + c;
    const int4 *cp = reinterpret_cast<const int4 *>(corners[h]);
    int tok[kS];
    float wv[kS];
#pragma unroll
    for (int i = 0; i < kS / 2; i++) {
        const int4 t = cp[i];
        tok[2 * i] = t.x;
        wv[2 * i] = __int_as_float(t.y);
        tok[2 * i + 1] = t.z;
        wv[2 * i + 1] = __int_as_float(t.w);
    }
    float v[kS];
#pragma unroll
    for (int i = 0; i < kS; i++) v[i] = vh[(int64_t)max(tok[i], 0) * ldv];
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kS; i++) acc = tok[i] >= 0 ? fmaf(wv[i], v[i], acc) : acc;
    out[(int64_t)q * kDM + h * kHD + c] = acc;
}

// ---------------------------------------------------------------------------
// mask -> box: per query, the bounding box of pixels with logit > 0 on the
// 200x200 mask, as inverse-sigmoid cxcywh normalised by 200.
__device__ __forceinline__ float invsig(float x) {
    x = fminf(fmaxf(x, 0.0f), 1.0f);
    const float x1 = fmaxf(x, 1e-5f);
    const float x2 = fmaxf(1.0f - x, 1e-5f);
    return logf(x1 / x2);
}

// the box of the block's (xmin, xmax, ymin, ymax) after the per-thread
// partials: wave shuffles, then wave 0's thread 0 over the 4 waves, then the
// inverse-sigmoid cxcywh normalised by 200 ((0, 0, 0, 0) for an empty mask)
__device__ __forceinline__ void box_finish(int xmin, int xmax, int ymin, int ymax, float *o) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        xmin = min(xmin, __shfl_xor(xmin, s));
        xmax = max(xmax, __shfl_xor(xmax, s));
        ymin = min(ymin, __shfl_xor(ymin, s));
        ymax = max(ymax, __shfl_xor(ymax, s));
    }
    __shared__ int red[4][4];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[wave][0] = xmin;
        red[wave][1] = xmax;
        red[wave][2] = ymin;
        red[wave][3] = ymax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) {
            xmin = min(xmin, red[w][0]);
            xmax = max(xmax, red[w][1]);
            ymin = min(ymin, red[w][2]);
            ymax = max(ymax, red[w][3]);
        }
        float bx0, by0, bx1, by1;
        if (xmax < 0) {
            bx0 = by0 = bx1 = by1 = 0.0f;
        } else {
            bx0 = (float)xmin;
            by0 = (float)ymin;
            bx1 = (float)xmax + 1.0f;
            by1 = (float)ymax + 1.0f;
        }
        bx0 /= (float)kMaskHW;
        bx1 /= (float)kMaskHW;
        by0 /= (float)kMaskHW;
        by1 /= (float)kMaskHW;
        const float cx = (bx0 + bx1) * 0.5f, cy = (by0 + by1) * 0.5f;
        const float bw = bx1 - bx0, bh = by1 - by0;
        o[0] = invsig(cx);
        o[1] = invsig(cy);
        o[2] = invsig(bw);
        o[3] = invsig(bh);
    }
}

__global__ __launch_bounds__(256) void k_mask_box(const float *__restrict__ ml,
                                                  float *__restrict__ out, int nq) {
    const int q = blockIdx.x;
    if (q >= nq) return;
    const float4 *m4 = reinterpret_cast<const float4 *>(ml + (int64_t)q * kMaskPix);
    int xmin = kMaskHW, xmax = -1, ymin = kMaskHW, ymax = -1;
    // 8 float4 loads in flight per thread and step (indices past the mask
    // clamped, their values ignored); branch-free integer min / max, exact
    // in any order
    constexpr int kN4 = kMaskPix / 4, kU = 8;
    for (int i0 = threadIdx.x; i0 < kN4; i0 += 256 * kU) {
        float4 v[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) v[u] = m4[min(i0 + u * 256, kN4 - 1)];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int i = i0 + u * 256;
            const int y = (4 * i) / kMaskHW, x = 4 * i - y * kMaskHW;  // 200 % 4 == 0: same row
            const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool pos = i < kN4 && e[j] > 0.0f;
                xmin = min(xmin, pos ? x + j : kMaskHW);
                xmax = max(xmax, pos ? x + j : -1);
                ymin = min(ymin, pos ? y : kMaskHW);
                ymax = max(ymax, pos ? y : -1);
            }
        }
    }
    box_finish(xmin, xmax, ymin, ymax, out + (int64_t)q * 4);
}

// mask -> box from sign bits: each thread takes words of 32 pixels; a word
// covers at most two rows of 200 (bits below `cut` on row y0, the rest on
// y0 + 1), and the first / last set bit of each part give its extreme
// columns.  Same min / max and the same finish as k_mask_box.
__global__ __launch_bounds__(256) void k_mask_box_bits(const uint32_t *__restrict__ bits, float *__restrict__ out,
                                                       int nq) {
    const int q = blockIdx.x;
    if (q >= nq) return;
    constexpr int kW = kMaskPix / 32;
    const uint32_t *bq = bits + (int64_t)q * kW;
    int xmin = kMaskHW, xmax = -1, ymin = kMaskHW, ymax = -1;
    for (int w = threadIdx.x; w < kW; w += 256) {
        const uint32_t v = bq[w];
        const int p0 = 32 * w, y0 = p0 / kMaskHW;
        const int cut = kMaskHW * (y0 + 1) - p0;  // >= 1
        const uint32_t lo = cut >= 32 ? v : (v & ((1u << cut) - 1u));
        const uint32_t hi = cut >= 32 ? 0u : (v & ~((1u << cut) - 1u));
        if (lo) {
            const int xb = p0 - kMaskHW * y0;
            xmin = min(xmin, xb + __builtin_ctz(lo));
            xmax = max(xmax, xb + 31 - __builtin_clz(lo));
            ymin = min(ymin, y0);
            ymax = max(ymax, y0);
        }
        if (hi) {
            const int xb = p0 - kMaskHW * (y0 + 1);
            xmin = min(xmin, xb + __builtin_ctz(hi));
            xmax = max(xmax, xb + 31 - __builtin_clz(hi));
            ymin = min(ymin, y0 + 1);
            ymax = max(ymax, y0 + 1);
        }
    }
    box_finish(xmin, xmax, ymin, ymax, out + (int64_t)q * 4);
}

// ---------------------------------------------------------------------------
// top-NQ tokens by max-class logit, descending, ties to the lower index.
// Each token gets a unique 64-bit key: order-preserving float bits (with -0
// folded into +0, since the CPU comparison treats them as equal) in the high
// word and the bit-inverted index in the low word, so "larger key" is exactly
// the CPU order.  A radix select over the key bytes finds a threshold with
// exactly NQ keys at or above it; those are gathered in LDS and each is placed
// by counting the gathered keys above it.  With a workspace, the keys are
// first computed by a grid-wide kernel.
constexpr int kTopkThreads = 1024;
constexpr int kTopkPer = 13;  // 13 * 1024 = 13312 >= 13125
constexpr int kTopkSort = 512;
constexpr int kTopkBins = 8192;  // histogram of the keys' top 13 bits (sign, exponent, 4 mantissa bits)
constexpr int kTopkCap = 1024;   // most keys the one-histogram path ranks directly

__device__ __forceinline__ uint64_t topk_key(float m, int idx) {
    m = m + 0.0f;  // -0 -> +0
    uint32_t u = __float_as_uint(m);
    u ^= (u >> 31) ? 0xFFFFFFFFu : 0x80000000u;
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ float row_max(const float *p, int nc) {
    float m = p[0];
    for (int c = 1; c < nc; c++) m = (m < p[c]) ? p[c] : m;
    return m;
}

// One key per token, over the whole grid (the selection kernel then reads
// 8 bytes per token instead of a row of logits).
__global__ __launch_bounds__(256) void k_topk_keys(const float *__restrict__ lg, uint64_t *__restrict__ keys,
                                                   int ntok, int nc) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t < ntok) keys[t] = topk_key(row_max(lg + (int64_t)t * nc, nc), t);
}

// keys == nullptr: the block computes the keys from the logits itself
__global__ __launch_bounds__(kTopkThreads) void k_topk(const float *__restrict__ lg,
                                                       const uint64_t *__restrict__ keys,
                                                       int32_t *__restrict__ out, int ntok, int nc,
                                                       int nq) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t whist[kTopkThreads / 64][256];
    __shared__ uint64_t sel[kTopkSort];
    __shared__ int s_digit, s_rank, s_cnt, s_done;
    __shared__ uint32_t fh[kTopkBins];
    __shared__ uint64_t fsel[kTopkCap];
    __shared__ uint32_t wsum[kTopkThreads / 64];
    __shared__ int s_fbin, s_ftot;
    const int tid = threadIdx.x;

    uint64_t key[kTopkPer];
#pragma unroll
    for (int j = 0; j < kTopkPer; j++) {
        const int t = tid + j * kTopkThreads;
        key[j] = 0;  // below every real key (real keys have a nonzero low word or high word)
        if (t < ntok) key[j] = keys ? keys[t] : topk_key(row_max(lg + (int64_t)t * nc, nc), t);
    }

    // One histogram over the keys' top 13 bits finds the bin that holds the
    // nq-th largest key.  Every key of a higher bin is selected; when those
    // and the threshold bin's keys number at most kTopkCap, they are gathered
    // and each is placed by counting the gathered keys above it: every key
    // above a gathered key is itself gathered, so that count is its rank.
    // More keys than that (scores that crowd into one bin) take the radix
    // select below.
    {
        const int lane = tid & 63, wv = tid >> 6;
        for (int i = tid; i < kTopkBins; i += kTopkThreads) fh[i] = 0;
        if (tid == 0) {
            s_fbin = -1;
            s_ftot = 0;
            s_cnt = 0;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kTopkPer; j++)
            if (key[j] != 0) atomicAdd(&fh[(uint32_t)(key[j] >> 51)], 1u);
        __syncthreads();
        // counts from the top bin down: thread tid owns bins B-1-8tid .. B-8-8tid
        constexpr int PB = kTopkBins / kTopkThreads;
        uint32_t cb[PB], tot = 0;
#pragma unroll
        for (int b = 0; b < PB; b++) {
            cb[b] = fh[kTopkBins - 1 - (tid * PB + b)];
            tot += cb[b];
        }
        uint32_t incl = tot;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t v = __shfl_up(incl, d);
            if (lane >= d) incl += v;
        }
        if (lane == 63) wsum[wv] = incl;
        __syncthreads();
        uint32_t run = incl - tot;
        for (int w = 0; w < wv; w++) run += wsum[w];
#pragma unroll
        for (int b = 0; b < PB; b++) {
            if (run < (uint32_t)nq && run + cb[b] >= (uint32_t)nq) {
                s_fbin = kTopkBins - 1 - (tid * PB + b);
                s_ftot = (int)(run + cb[b]);
            }
            run += cb[b];
        }
        __syncthreads();
        const int fbin = s_fbin, ftot = s_ftot;
        if (fbin >= 0 && ftot <= kTopkCap) {
#pragma unroll
            for (int j = 0; j < kTopkPer; j++) {
                if (key[j] != 0 && (int)(uint32_t)(key[j] >> 51) >= fbin) fsel[atomicAdd(&s_cnt, 1)] = key[j];
            }
            __syncthreads();
            for (int i = tid; i < ftot; i += kTopkThreads) {
                const uint64_t ki = fsel[i];
                int r = 0;
                for (int j = 0; j < ftot; j++) r += fsel[j] > ki ? 1 : 0;
                if (r < nq) out[r] = (int32_t)(0xFFFFFFFFu - (uint32_t)(ki & 0xFFFFFFFFu));
            }
            return;
        }
        __syncthreads();  // s_cnt is reused below
    }

    // Radix select, most significant byte first.  Each pass histograms the
    // byte of the keys that still match the selected prefix; each wave counts
    // into a histogram of its own (nearly all keys share their top bytes, and
    // one shared histogram serialises those atomics over the whole block).
    // The pass that lands on a bin holding exactly the remaining rank ends
    // the search: every key of that bin is selected, so the threshold is the
    // prefix with its lower bytes zero.
    constexpr int kWaves = kTopkThreads / 64;
    uint32_t *wh = &whist[0][0];
    const int wave = tid >> 6;
    uint64_t prefix = 0, mask = 0;
    int rank = nq;  // 1-based rank still to find within the current prefix
    for (int byte = 7; byte >= 0; byte--) {
        for (int i = tid; i < kWaves * 256; i += kTopkThreads) wh[i] = 0;
        __syncthreads();
        const int sh = byte * 8;
#pragma unroll
        for (int j = 0; j < kTopkPer; j++)
            if ((key[j] & mask) == prefix && key[j] != 0) atomicAdd(&whist[wave][(key[j] >> sh) & 0xFF], 1u);
        __syncthreads();
        if (tid < 256) {
            uint32_t c = 0;
#pragma unroll
            for (int w = 0; w < kWaves; w++) c += whist[w][tid];
            hist[tid] = c;
        }
        __syncthreads();
        if (tid < 64) {
            // wave 0 scans the 256 bins from the top: 4 bins per lane
            uint32_t c4[4], tot = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                c4[b] = hist[255 - (tid * 4 + b)];
                tot += c4[b];
            }
            uint32_t incl = tot;  // inclusive prefix over lanes (top bins first)
#pragma unroll
            for (int s = 1; s < 64; s <<= 1) {
                const uint32_t v = __shfl_up(incl, s);
                if (tid >= s) incl += v;
            }
            uint32_t run = incl - tot;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (run < (uint32_t)rank && run + c4[b] >= (uint32_t)rank) {
                    s_digit = 255 - (tid * 4 + b);
                    s_rank = rank - (int)run;
                    s_done = c4[b] == (uint32_t)(rank - (int)run);
                }
                run += c4[b];
            }
        }
        __syncthreads();
        prefix |= (uint64_t)s_digit << sh;
        mask |= (uint64_t)0xFF << sh;
        rank = s_rank;
        const int done = s_done;
        __syncthreads();
        if (done) break;
    }

    // gather keys >= threshold (exactly nq of them: keys are unique)
    if (tid == 0) s_cnt = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTopkPer; j++) {
        if (key[j] != 0 && key[j] >= prefix) {
            const int pos = atomicAdd(&s_cnt, 1);
            if (pos < kTopkSort) sel[pos] = key[j];
        }
    }
    __syncthreads();

    // each selected key's position is the number of selected keys above it
    const int cnt = min(s_cnt, kTopkSort);
    for (int i = tid; i < cnt; i += kTopkThreads) {
        const uint64_t ki = sel[i];
        int r = 0;
        for (int j = 0; j < cnt; j++) r += sel[j] > ki ? 1 : 0;
        if (r < nq) out[r] = (int32_t)(0xFFFFFFFFu - (uint32_t)(ki & 0xFFFFFFFFu));
    }
}

}  // namespace

hipError_t msdeform(const float *val, int ldv, const float *off, int ldo, const float *awr, int ldw,
                    const float *ref, float *out, int nq, hipStream_t s) {
    hipLaunchKernelGGL(k_msdeform, dim3(nq), dim3(256), 0, s, val, off, awr, ref, out, nq, ldv, ldo, ldw);
    return hipGetLastError();
}

hipError_t mask_box(const float *ml, float *out, int nq, hipStream_t s) {
    hipLaunchKernelGGL(k_mask_box, dim3(nq), dim3(256), 0, s, ml, out, nq);
    return hipGetLastError();
}

hipError_t mask_box_bits(const uint32_t *bits, float *out, int nq, hipStream_t s) {
    hipLaunchKernelGGL(k_mask_box_bits, dim3(nq), dim3(256), 0, s, bits, out, nq);
    return hipGetLastError();
}

hipError_t topk(const float *logits, int32_t *out, int ntok, int nc, int nq, void *ws, int64_t ws_bytes,
                hipStream_t s) {
    uint64_t *keys = nullptr;
    if (ws && ws_bytes >= (int64_t)ntok * 8) {
        keys = (uint64_t *)ws;
        hipLaunchKernelGGL(k_topk_keys, dim3((ntok + 255) / 256), dim3(256), 0, s, logits, keys, ntok, nc);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(kTopkThreads), 0, s, logits, keys, out, ntok, nc, nq);
    return hipGetLastError();
}

}  // namespace ppdl
