// PP-DocLayoutV3 on MI355X: the reference's graph (src/ppdoclayout.cpp:363-883)
// rebuilt as a list of kernel launches over device buffers, captured once
// into a hipGraph and replayed per image.
//
//  * Weights come from the reference's GGUF (F32, BN folded) and are repacked
//    at load (src/ppdoclayout.cpp:251-346) through ppdl_hip_repack_conv.
//  * Every conv goes through the tagged-op C-ABI (ppdl_hip_run), chosen by
//    the same router as builder::conv (src/ppdoclayout.cpp:388-543): 1x1 ->
//    op 14, k3 s1 p1 -> ops 15/12/11 (F(4,3)), k2 / k3 s2 -> op 16,
//    depthwise -> the stock depthwise kernel.  MSDeformAttn, mask->box and
//    top-300 are ops 2, 1 and 13.
//  * Stock ops (linears, layer norm, attention, interpolation, ...) use this
//    library's own kernels; concats cost nothing: producers write straight
//    into their channel slice of the concatenated buffer.
#include <hip/hip_runtime.h>
#include <sys/stat.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "../../include/ppdl_hip_ops.h"
#include "../../include/ppdoclayout.h"
#include "gguf.h"
#include "net_internal.h"

namespace ppdl {
namespace {

constexpr int IMG = 800, NQ = 300, NC = 25, NTOK = kNTOK, NPIX = kMaskPix;

struct Img {
    float *d = nullptr;
    int C = 0, H = 0, W = 0;
    int64_t ld = 0;  // channel-plane stride in floats; 0: H * W (packed planes)
    int64_t plane() const { return ld ? ld : (int64_t)H * W; }
};
struct Seq {
    float *d = nullptr;
    int T = 0, D = 0, ld = 0;  // token-major rows of D features, row stride ld
};

struct Node {
    std::string name;
    int kernels;  // device kernels this node launches
    std::function<int(hipStream_t)> run;
    int lane = 0;  // stream the node runs on (0 = the graph's main stream)
    int kind = 0;  // 0 kernels, 1 fork (lane waits for main), 2 join (main waits for lane)
    int ev = -1;   // fork / join: index of its event
    int cls = 0;         // 0 other, 1 conv GEMM, 2 linear GEMM
    double flops = 0.0;  // algorithmic GEMM FLOP per run
    double bytes = 0.0;  // compulsory GEMM operand bytes per run
    std::string kern;    // GEMM kernel(s) the node's plan launches
};

struct DumpRec {
    std::string name;
    const void *d;
    std::vector<int64_t> ne;
    bool i32;
};

bool ends_with(const std::string &s, const char *suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

ppdl_tview view(const void *d, std::vector<int64_t> ne, int32_t type = PPDL_TYPE_F32) {
    ppdl_tview v;
    v.data = const_cast<void *>(d);
    while (ne.size() < 4) ne.push_back(1);
    int64_t nb = 4;
    for (int i = 0; i < 4; i++) {
        v.ne[i] = ne[i];
        v.nb[i] = nb;
        nb *= ne[i];
    }
    v.type = type;
    return v;
}
ppdl_tview view(const Img &x) {
    ppdl_tview v = view(x.d, {x.W, x.H, x.C});
    v.nb[2] = x.plane() * 4;
    v.nb[3] = v.nb[2] * x.C;
    return v;
}

// Winograd planes ne(T, C, 36) with rows padded to ldt tiles
ppdl_tview planes(const float *d, int64_t T, int64_t C, int64_t ldt) {
    ppdl_tview v = view(d, {T, C, 36});
    v.nb[1] = ldt * 4;
    v.nb[2] = v.nb[1] * C;
    v.nb[3] = v.nb[2] * 36;
    return v;
}

// ne(cols, rows) rows of `cols` floats, `ld` floats apart (a column slice of
// a wider row-major matrix)
ppdl_tview row_view(const float *d, int64_t cols, int64_t rows, int64_t ld) {
    ppdl_tview v = view(d, {cols, rows});
    v.nb[1] = ld * 4;
    v.nb[2] = v.nb[3] = v.nb[1] * rows;
    return v;
}

std::vector<int32_t> op_params(int op, int p14, int p15) {
    std::vector<int32_t> v(16, 0);
    v[11] = (int32_t)PPDL_WG4_SET;  // every .wg4 here comes from ppdl_hip_repack_conv
    v[12] = (int32_t)PPDL_MAGIC;
    v[13] = op;
    v[14] = p14;
    v[15] = p15;
    return v;
}

alignas(16) const float kShapeOnly[4] = {0.0f, 0.0f, 0.0f, 0.0f};

class Net {
   public:
    ~Net() {
        if (exec_) (void)hipGraphExecDestroy(exec_);
        if (graph_) (void)hipGraphDestroy(graph_);
        for (hipEvent_t e : events_) (void)hipEventDestroy(e);
        for (int l = 1; l < kLanes; l++)
            if (lanes_[l]) (void)hipStreamDestroy(lanes_[l]);
        if (stream_) (void)hipStreamDestroy(stream_);
        for (void *p : allocs_) (void)hipFree(p);
    }

    bool load(const std::string &path, std::string *err);
    bool fold_repvgg(GgufFile &g, const std::string &bp, std::string *err);
    bool concat_conv1x1(GgufFile &g, const std::vector<std::string> &parts, const std::string &name,
                        std::string *err);
    bool concat_linears(GgufFile &g, const std::vector<std::string> &parts, const std::string &name,
                        std::string *err);
    bool build(bool dumps, std::string *err);
    bool capture(std::string *err);
    int replay();  // one graph launch + sync
    double time_graph(int iters);
    int profile_nodes(int iters, ppdl_node_stat *out, int cap);
    int profile_in_graph(int reps, ppdl_node_stat *out, int cap);
    bool upload_image(const float *host);
    // the host result's inputs: mask sign bits packed on the device, then
    // logits, boxes, order and the bits copied into pinned buffers
    bool download(float *logits, float *boxes, float *order, uint32_t *mbits);
    bool mask_logits();  // masks_ = the final mask logits of the last replay

    int nodes() const {
        int k = 0;
        for (const auto &n : nodes_) k += n.kernels;
        return k;
    }

    // outputs
    float *logits_ = nullptr, *boxes_ = nullptr, *order_ = nullptr, *masks_ = nullptr, *refu_ = nullptr;
    int32_t *topk_ = nullptr;
    uint32_t *mbits_ = nullptr;  // sign bits of the final mask logits, written by the graph
    GemmArgs mask_logits_{};     // the final mask logits into masks_ (run on request, not in the graph)
    std::vector<DumpRec> dumps_;

   private:
    // ---- memory ----
    // Buffers and weights are carved out of 256 MiB chunks (256-byte
    // aligned, never freed before the context): a few large allocations
    // instead of hundreds of small ones, so the graph's working set sits in
    // few, large mappings.  Larger requests, and every request with
    // PPDL_ARENA=0, get an allocation of their own.
    static constexpr size_t kChunk = (size_t)256 << 20;
    float *alloc(int64_t nfloat) {
        const size_t bytes = ((size_t)std::max<int64_t>(nfloat, 1) * 4 + 255) & ~(size_t)255;
        const char *ea = getenv("PPDL_ARENA");
        const bool arena = !(ea && ea[0] == '0');
        void *p = nullptr;
        if (arena && bytes <= kChunk) {
            if (bytes > chunk_left_) {
                if (hipMalloc(&p, kChunk) != hipSuccess) {
                    oom_ = true;
                    return nullptr;
                }
                allocs_.push_back(p);
                chunk_ = (char *)p;
                chunk_left_ = kChunk;
            }
            float *r = (float *)chunk_;
            chunk_ += bytes;
            chunk_left_ -= bytes;
            return r;
        }
        if (hipMalloc(&p, bytes) != hipSuccess) {
            oom_ = true;
            return nullptr;
        }
        allocs_.push_back(p);
        return (float *)p;
    }
    float *upload(const std::vector<float> &h) {
        float *d = alloc((int64_t)h.size());
        if (d && hipMemcpy(d, h.data(), h.size() * 4, hipMemcpyHostToDevice) != hipSuccess) oom_ = true;
        return d;
    }
    const float *W(const std::string &name) {
        auto it = w_.find(name);
        if (it == w_.end()) {
            if (missing_.empty()) missing_ = name;
            return nullptr;
        }
        return it->second;
    }
    const std::vector<int64_t> &shape(const std::string &name) {
        static const std::vector<int64_t> none = {1, 1, 1, 1};
        auto it = ne_.find(name);
        if (it == ne_.end()) {
            if (missing_.empty()) missing_ = name;
            return none;
        }
        return it->second;
    }
    void dump(const char *name, const void *d, std::vector<int64_t> ne, bool i32 = false) {
        if (want_dumps_) dumps_.push_back({name, d, ne, i32});
    }
    void dump(const char *name, const Img &x) { dump(name, x.d, {x.W, x.H, x.C}); }

    // ---- node emission ----
    void node(const std::string &name, int kernels, std::function<int(hipStream_t)> fn) {
        if (pend_.on) flush_pending();
        nodes_.push_back({name, kernels, std::move(fn)});
        nodes_.back().lane = lane_;
    }
    // A Winograd conv's output transform is held back until the next node:
    // when that is the input transform of a Winograd conv on exactly this
    // output, both become one chained node (wg4_chain); before any other
    // node it is emitted as op 11.  Opt-in (PPDL_WG_CHAIN=1): the 13 chains
    // of the network (stage 2's layer chain, the RepVGG chains of the four
    // CSP layers) remove 13 launches, yet the graph replayed 6-10 us slower
    // (same-process A/B, bands of 4 and 8 tile rows): the recomputed halo
    // rows and the kernel's two dependent phases cost what the launch saved.
    struct Scratch;
    struct PendOut {
        bool on = false;
        std::string name;
        Img y;
        const float *bias = nullptr, *add = nullptr;
        int act = 0, add_mode = 0, ldt = 0, TW = 0, TH = 0;
        Scratch *sc = nullptr;
        std::vector<int32_t> p_out;
    };
    PendOut pend_;
    void flush_pending() {
        const PendOut pp = pend_;
        pend_.on = false;
        Scratch *sc = pp.sc;
        const int T = pp.TW * pp.TH, OC = pp.y.C, OW = pp.y.W, OH = pp.y.H;
        node(pp.name + ".wg_out", 1, [=](hipStream_t st) {
            ppdl_tview d = view(pp.y);
            ppdl_tview sv[3] = {planes(sc->yt, T, OC, pp.ldt), view(pp.bias, {OC}), view(pp.add, {OW, OH, OC})};
            return ppdl_hip_run(pp.p_out.data(), &d, sv, pp.add_mode ? 3 : 2, st);
        });
    }
    // Independent branches: fork(l) makes lane l wait for everything emitted
    // so far on the main lane and directs the following nodes to lane l;
    // main() directs them back without a dependency; join(l) makes the main
    // lane wait for everything lane l has been given.  Each lane has its own
    // scratch (F(4,3) planes, split-K workspace), so branches never share it.
    void fork(int l) {
        if (!multi_lane_) return;
        sync_node("fork", 1, l);
        lane_ = l;
    }
    void main_lane() { lane_ = 0; }
    void join(int l) {
        if (!multi_lane_) return;
        sync_node("join", 2, l);
        lane_ = 0;
    }
    void sync_node(const char *nm, int kind, int l) {
        if (pend_.on) flush_pending();
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            if (bad_node_.empty()) bad_node_ = nm;
            return;
        }
        events_.push_back(e);
        Node n{std::string(nm) + std::to_string(l), 0, nullptr};
        n.lane = l;
        n.kind = kind;
        n.ev = (int)events_.size() - 1;
        nodes_.push_back(std::move(n));
    }
    int launch_all();  // every node, on its lane, in list order
    // GEMM bookkeeping of the node just emitted (for ppdl_profile_nodes)
    void gemm_meta(int cls, const GemmArgs &g, int64_t ws_bytes, bool im2col) {
        Node &n = nodes_.back();
        n.cls = cls;
        n.flops = 2.0 * g.M * (double)g.N * g.K * g.batch;
        // the implicit-im2col B is the input image, read once
        const double b_elems = im2col ? (double)g.IC * g.IH * g.IW : (double)g.K * g.N;
        n.bytes = 4.0 * g.batch * ((double)g.M * g.K + b_elems + (g.bits ? g.M * (double)g.N / 32.0 : (double)g.M * g.N));
        n.kern = gemm_kernel_name(g, ws_bytes, im2col);
    }
    // one tagged op through the C-ABI; a GEMM op gets the shared split-K
    // workspace appended when its plan asks for one
    void tagged(const std::string &name, int op, int p14, int p15, ppdl_tview dst, std::vector<ppdl_tview> src) {
        const std::vector<int32_t> pv = op_params(op, p14, p15);
        const int64_t wsb = ppdl_hip_workspace_bytes(pv.data(), &dst, src.data(), (int)src.size());
        if (wsb < 0) {
            if (bad_node_.empty()) bad_node_ = name;
            return;
        }
        Scratch *sc = &sc_[lane_];
        sc->ws_need = std::max(sc->ws_need, wsb);
        const int kernels = (op == PPDL_OP_WG4_INPUT_PAD || op == PPDL_OP_WG4_OUTPUT) ? 1 : (wsb > 0 ? 2 : 1);
        node(name, kernels, [sc, pv, dst, src, wsb](hipStream_t s) {
            std::vector<ppdl_tview> sv = src;
            if (wsb > 0) sv.push_back(view(sc->ws, {(sc->ws_bytes + 3) / 4}));
            return ppdl_hip_run(pv.data(), &dst, sv.data(), (int)sv.size(), s);
        });
        GemmArgs g;
        bool im2col;
        if (gemm_args_of(pv.data(), &dst, src.data(), &g, &im2col)) gemm_meta(1, g, wsb, im2col);
    }
    // cls: 2 linear (token-major) GEMM, 1 a conv that writes token-major
    void gemm(const std::string &name, GemmArgs g, int cls = 2) {
        const int64_t wsb = gemm_ws_bytes_for(g, false);
        Scratch *sc = &sc_[lane_];
        sc->ws_need = std::max(sc->ws_need, wsb);
        node(name, wsb > 0 ? 2 : 1, [sc, g, wsb](hipStream_t s) {
            GemmWorkspace ws{wsb > 0 ? sc->ws : nullptr, wsb > 0 ? sc->ws_bytes : 0};
            return gemm_dense(g, ws, s) == hipSuccess ? 0 : 3;
        });
        gemm_meta(cls, g, wsb, false);
    }
    static int ok(hipError_t e) { return e == hipSuccess ? 0 : 3; }

    // ---- layers ----
    // out_ld: channel-plane stride of the output (0: packed); depthwise and
    // 1x1 convs only, like a strided x
    Img conv(const Img &x, const std::string &name, int s, int p, int act, float *out = nullptr, int pad_end = 0,
             const float *add = nullptr, int add_mode = 0, int64_t out_ld = 0);
    // ln: a layer norm applied to x in the GEMM's A loader, its result
    // stored to ln_out
    Seq lin(const Seq &x, const std::string &name, int act, float *out = nullptr, const float *add = nullptr,
            int add_mode = 0, const float *a_add = nullptr, int a_add_n = 0, const std::string &ln = "",
            float *ln_out = nullptr);
    Seq ln(const Seq &a, const float *b, const std::string &name, float *out = nullptr, int out_chw = 0);
    Seq mlp3(const Seq &x, const std::string &pfx);
    Seq lin_in4(const Seq &x, const std::string &first, const std::string &second, int act,
                const Seq *box_h = nullptr, float *box_out = nullptr);
    Seq mha(const Seq &x, const float *pos, const std::string &pfx, float *out, const float *resid);
    void hg_block(const Img &cat, int cin, const std::string &pfx, bool light, int mid, Img *y, float *out,
                  const float *resid);
    Img csp(const Img &x, const std::string &pfx, float *out);

    std::vector<void *> allocs_;
    char *chunk_ = nullptr;  // next free byte of the current chunk
    size_t chunk_left_ = 0;
    std::map<std::string, float *> w_;
    std::map<std::string, std::vector<int64_t>> ne_;
    std::vector<Node> nodes_;
    std::string missing_, bad_node_, failed_;
    bool oom_ = false, want_dumps_ = false;
    // per-lane scratch shared by that lane's nodes (they run in order)
    struct Scratch {
        int64_t ws_need = 0, ws_bytes = 0;  // split-K / top-k workspace
        void *ws = nullptr;
        int64_t wg_need = 0;  // F(4,3) dt / yt planes
        float *dt = nullptr, *yt = nullptr;
    };
    static constexpr int kLanes = 3;
    Scratch sc_[kLanes];
    int lane_ = 0;
    // Branches on separate streams (PPDL_GRAPH_LANES=1).  Off by default:
    // measured on MI355X / ROCm 7, the captured graph with two side branches
    // replays ~0.1 ms slower than the same nodes on one stream, more than
    // the ~0.2 ms of overlappable work it gains (the value projection's
    // branch alone: ~0.15 ms slower).
    bool multi_lane_ = false;
    hipStream_t lanes_[kLanes] = {};  // lanes_[0] is stream_
    std::vector<hipEvent_t> events_;
    hipStream_t stream_ = nullptr;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
    float *image_ = nullptr, *pos_ = nullptr, *valid_ = nullptr;
};

// ---------------------------------------------------------------------------
// Loading: read every tensor, repack conv weights (.wr [tap][ic][oc] and, for
// 3x3, the 36-plane .wg4), store linear weights transposed (.wt [in][out])
// for the row-major-activation GEMM, keep biases / norms / depthwise weights
// as they are.  Linears that share their input are also stored side by side
// (concat_linears).
bool Net::load(const std::string &path, std::string *err) {
    GgufFile g;
    if (!gguf_open(path, &g, err)) return false;
    std::vector<float> h;
    for (const auto &t : g.tensors) {
        h.resize((size_t)t.nelem());
        if (!gguf_read_f32(g, t, h.data(), err)) return false;
        ne_[t.name] = t.ne;
        const std::string base = ends_with(t.name, ".weight") ? t.name.substr(0, t.name.size() - 7) : "";
        if (!base.empty() && t.ne.size() == 4 && t.ne[3] > 1 && t.ne[2] > 1 && t.ne[0] == t.ne[1] &&
            t.ne[0] <= 3) {
            const int64_t K = t.ne[0], IC = t.ne[2], OC = t.ne[3];
            std::vector<float> wr((size_t)(K * K * IC * OC)), wg4(K == 3 ? (size_t)(36 * IC * OC) : 0);
            if (ppdl_hip_repack_conv(h.data(), OC, IC, K, wr.data(), K == 3 ? wg4.data() : nullptr) != PPDL_OK) {
                *err = "repack failed: " + t.name;
                return false;
            }
            w_[base + ".wr"] = upload(wr);
            if (K == 3) w_[base + ".wg4"] = upload(wg4);
        } else if (!base.empty() && t.ne.size() == 2) {
            const int64_t in = t.ne[0], out = t.ne[1];
            std::vector<float> wt((size_t)(in * out));
            for (int64_t o = 0; o < out; o++)
                for (int64_t i = 0; i < in; i++) wt[(size_t)(i * out + o)] = h[(size_t)(o * in + i)];
            w_[base + ".wt"] = upload(wt);
        } else {
            w_[t.name] = upload(h);
        }
        if (oom_) {
            *err = "device allocation failed while loading " + t.name;
            return false;
        }
    }
    // Linears that read the same input run as one GEMM over their weights
    // stored side by side: q|k|v of each attention, the decoder's sampling
    // offsets | attention logits, and the six decoder layers' value
    // projections of the encoder tokens.
    for (const std::string a : {"aifi", "dec0.sa", "dec1.sa", "dec2.sa", "dec3.sa", "dec4.sa", "dec5.sa"})
        if (!concat_linears(g, {a + ".q", a + ".k", a + ".v"}, a + ".qkv", err)) return false;
    for (int i = 0; i < 6; i++) {
        const std::string d = "dec" + std::to_string(i) + ".ca";
        if (!concat_linears(g, {d + ".so", d + ".aw"}, d + ".soaw", err)) return false;
    }
    {
        std::vector<std::string> vp;
        for (int i = 0; i < 6; i++) vp.push_back("dec" + std::to_string(i) + ".ca.vp");
        if (!concat_linears(g, vp, "dec.ca.vp", err)) return false;
    }
    for (const std::string blk : {"fpn0", "fpn1", "pan0", "pan1"}) {
        for (int i = 0; i < 3; i++)
            if (!fold_repvgg(g, blk + ".bn" + std::to_string(i), err)) return false;
        if (!concat_conv1x1(g, {blk + ".c1", blk + ".c2"}, blk + ".c12", err)) return false;
    }
    if (oom_) {
        *err = "device allocation failed";
        return false;
    }
    return true;
}

// RepVGG block bp (src/ppdoclayout.cpp:656-660): silu(c1_3x3(a) + c2_1x1(a))
// is one 3x3 conv whose centre tap carries both branches, w = c1.w with
// w[oc][ic][1][1] += c2.w[oc][ic], bias c1.b + c2.b: the same sums
// regrouped, so the block becomes a single Winograd conv and its 1x1 GEMM
// disappears.  Stored as bp.rep (.wr, .wg4, .bias, shape); skipped (the
// graph keeps the two convs) when a part is absent or the shapes differ.
bool Net::fold_repvgg(GgufFile &g, const std::string &bp, std::string *err) {
    const std::string c1 = bp + ".c1", c2 = bp + ".c2";
    for (const auto &n : {c1 + ".weight", c1 + ".bias", c2 + ".weight", c2 + ".bias"})
        if (!g.index.count(n)) return true;
    const auto &t1 = g.tensors[g.index[c1 + ".weight"]], &t2 = g.tensors[g.index[c2 + ".weight"]];
    if (t1.ne.size() != 4 || t2.ne.size() != 4 || t1.ne[0] != 3 || t1.ne[1] != 3 || t2.ne[0] != 1 || t2.ne[1] != 1 ||
        t1.ne[2] != t2.ne[2] || t1.ne[3] != t2.ne[3])
        return true;
    const int64_t IC = t1.ne[2], OC = t1.ne[3];
    std::vector<float> w((size_t)(9 * IC * OC)), w2((size_t)(IC * OC)), b1((size_t)OC), b2((size_t)OC);
    if (!gguf_read_f32(g, t1, w.data(), err) || !gguf_read_f32(g, t2, w2.data(), err) ||
        !gguf_read_f32(g, g.tensors[g.index[c1 + ".bias"]], b1.data(), err) ||
        !gguf_read_f32(g, g.tensors[g.index[c2 + ".bias"]], b2.data(), err))
        return false;
    for (int64_t o = 0; o < OC; o++) {
        for (int64_t i = 0; i < IC; i++) w[(size_t)((o * IC + i) * 9 + 4)] += w2[(size_t)(o * IC + i)];  // [oc][ic][kh][kw]
        b1[(size_t)o] += b2[(size_t)o];
    }
    std::vector<float> wr((size_t)(9 * IC * OC)), wg4((size_t)(36 * IC * OC));
    if (ppdl_hip_repack_conv(w.data(), OC, IC, 3, wr.data(), wg4.data()) != PPDL_OK) {
        *err = "repack failed: " + bp + ".rep";
        return false;
    }
    w_[bp + ".rep.wr"] = upload(wr);
    w_[bp + ".rep.wg4"] = upload(wg4);
    w_[bp + ".rep.bias"] = upload(b1);
    ne_[bp + ".rep.weight"] = t1.ne;
    return true;
}

// 1x1 convs `parts` over the same input (weights ne(1, 1, IC, OC_i)) stored
// as one conv `name` whose output channels are the parts' in order (.wr,
// .bias, shape): one GEMM instead of one per part, the same sums.  Skipped
// (no entry) when a part is absent or not a 1x1 conv over IC.
bool Net::concat_conv1x1(GgufFile &g, const std::vector<std::string> &parts, const std::string &name,
                         std::string *err) {
    int64_t IC = -1, total = 0;
    for (const auto &p : parts) {
        if (!g.index.count(p + ".weight") || !g.index.count(p + ".bias")) return true;
        const auto &t = g.tensors[g.index[p + ".weight"]];
        if (t.ne.size() != 4 || t.ne[0] != 1 || t.ne[1] != 1 || (IC >= 0 && t.ne[2] != IC)) return true;
        if (g.tensors[g.index[p + ".bias"]].nelem() != t.ne[3]) return true;
        IC = t.ne[2];
        total += t.ne[3];
    }
    std::vector<float> w((size_t)(IC * total)), b((size_t)total);
    int64_t o0 = 0;
    for (const auto &p : parts) {
        const auto &t = g.tensors[g.index[p + ".weight"]];
        // [oc][ic] rows of the part follow the previous parts' rows
        if (!gguf_read_f32(g, t, w.data() + o0 * IC, err) ||
            !gguf_read_f32(g, g.tensors[g.index[p + ".bias"]], b.data() + o0, err))
            return false;
        o0 += t.ne[3];
    }
    std::vector<float> wr((size_t)(IC * total));
    if (ppdl_hip_repack_conv(w.data(), (int)total, (int)IC, 1, wr.data(), nullptr) != PPDL_OK) {
        *err = "repack failed: " + name;
        return false;
    }
    w_[name + ".wr"] = upload(wr);
    w_[name + ".bias"] = upload(b);
    ne_[name + ".weight"] = {1, 1, IC, total};
    return true;
}

// Linears `parts` (weights ne(in, out_i), biases ne(out_i)) stored as one
// transposed weight [in][sum out_i] and one bias under `name`.  Skipped (no
// entry; the graph build then reports the missing weight) when a part is
// absent or the input widths differ.
bool Net::concat_linears(GgufFile &g, const std::vector<std::string> &parts, const std::string &name,
                         std::string *err) {
    int64_t in = -1, total = 0;
    for (const auto &p : parts) {
        if (!g.index.count(p + ".weight") || !g.index.count(p + ".bias")) return true;
        const auto &t = g.tensors[g.index[p + ".weight"]];
        if (t.ne.size() != 2 || (in >= 0 && t.ne[0] != in)) return true;
        if (g.tensors[g.index[p + ".bias"]].nelem() != t.ne[1]) return true;
        in = t.ne[0];
        total += t.ne[1];
    }
    std::vector<float> wt((size_t)(in * total)), b((size_t)total), h;
    int64_t o0 = 0;
    for (const auto &p : parts) {
        const auto &t = g.tensors[g.index[p + ".weight"]];
        const int64_t out = t.ne[1];
        h.resize((size_t)(in * out));
        if (!gguf_read_f32(g, t, h.data(), err) || !gguf_read_f32(g, g.tensors[g.index[p + ".bias"]], b.data() + o0, err))
            return false;
        for (int64_t o = 0; o < out; o++)
            for (int64_t i = 0; i < in; i++) wt[(size_t)(i * total + o0 + o)] = h[(size_t)(o * in + i)];
        o0 += out;
    }
    w_[name + ".wt"] = upload(wt);
    w_[name + ".bias"] = upload(b);
    ne_[name + ".weight"] = {in, total};
    return true;
}

// k3 s1 p1 convs with at most 48 output channels on a large map run as the
// fused Winograd kernel (op 17), the rest as the three-op pipeline 15 -> 12
// -> 11.  Each op 17 block walks every input channel 4 at a time and
// recomputes the input transform per 16-channel output tile, so it wins only
// where the 3-op pipeline's plane traffic and launches dominate: in the
// network graph 48 -> 48 @200 takes 26 us against 33.5; 96 -> 96 @100 (26.5
// vs 24.8 us), 64 -> 64 @200 (52.9 vs 39.1) and every 256-channel conv (61 vs
// 20-63 us in isolation) are faster as three ops.  PPDL_WG_FUSED=0 / 1 forces
// either path for every k3 s1 p1 conv (read at graph build).
// With the kernel's unmasked-weight form and whole prefetch groups, 96- and
// 128-channel inputs to 96 outputs at 100x100 (stage 1's six convs) also
// favour it in isolation: 96 -> 96 25.4 against 30.7 us, 128 -> 96 33.3
// against 35.8 us (64 -> 64 @100 21.2 / 21.8); 64 -> 64 and 128 -> 64 @200
// stay three ops.  PPDL_WG_FUSED_WIDE=0 keeps only the 48-channel rule.
bool wg_fused(int IC, int H, int W, int OC) {
    if (const char *e = getenv("PPDL_WG_FUSED")) return e[0] == '1';
    const int64_t T = (int64_t)((W + 3) / 4) * ((H + 3) / 4);
    const char *ew = getenv("PPDL_WG_FUSED_WIDE");
    const bool wide = !(ew && ew[0] == '0') && IC <= 128 && OC <= 96 && T >= 625 && T <= 1024;
    return (IC <= 96 && OC <= 48 && T >= 625) || wide;
}

// ---------------------------------------------------------------------------
// builder::conv (src/ppdoclayout.cpp:388-543): route by shape.
Img Net::conv(const Img &x, const std::string &name, int s, int p, int act, float *out, int pad_end,
              const float *add, int add_mode, int64_t out_ld) {
    const auto &ne = shape(name + ".weight");  // (K, K, IC, OC)
    const int K = (int)ne[0], ICw = (int)ne[2], OC = (int)ne[3];
    const float *b = W(name + ".bias");
    const int OH = (x.H + 2 * p + pad_end - K) / s + 1, OW = (x.W + 2 * p + pad_end - K) / s + 1;
    const int64_t ypl = out_ld ? out_ld : (int64_t)OH * OW;
    Img y{out ? out : alloc((int64_t)OC * ypl), OC, OH, OW, out_ld};
    if (ICw == 1 && x.C != 1) {
        // depthwise: ggml_conv_2d_dw_direct + bias + act (:400-404)
        const float *w = W(name + ".weight");
        const Img xi = x;
        node(name, 1, [=](hipStream_t st) {
            return ok(dwconv(xi.d, w, b, y.d, xi.C, xi.H, xi.W, K, s, p, act, xi.plane(), y.plane(), st));
        });
        return y;
    }
    if (ICw != x.C && bad_node_.empty()) bad_node_ = name + " (channel mismatch)";
    // plane-strided maps exist for the 1x1 GEMMs only (ops 3 / 14 take them)
    if ((x.ld || out_ld) && !(K == 1 && s == 1 && p == 0 && pad_end == 0) && bad_node_.empty())
        bad_node_ = name + " (plane-strided map into a conv other than 1x1)";
    const ppdl_tview vb = view(b, {OC});
    if (K == 1 && s == 1 && p == 0 && pad_end == 0) {
        // op 3 + op 5 fused: one GEMM writing CHW with bias/act (:408-423)
        std::vector<ppdl_tview> src = {view(x), view(W(name + ".wr"), {OC, x.C, 1}), vb};
        if (add_mode) src.push_back(view(add, {OW, OH, OC}));
        tagged(name, PPDL_OP_CONV1X1_BA, act, add_mode, view(y), src);
    } else if (K == 3 && s == 1 && p == 1 && pad_end == 0 && add_mode == 0 && wg_fused(x.C, x.H, x.W, OC)) {
        // Winograd F(4,3) (:425-463) as one kernel (op 17): input transform,
        // 36 plane products and output transform + bias + act, no planes in HBM
        const size_t before = nodes_.size();
        tagged(name, PPDL_OP_WG4_CONV, act, 0, view(y), {view(x), view(W(name + ".wg4"), {OC, x.C, 36}), vb});
        if (nodes_.size() > before) {
            Node &n = nodes_.back();
            const double T = (double)((OW + 3) / 4) * ((OH + 3) / 4);
            n.cls = 1;
            n.flops = 2.0 * 36.0 * OC * T * x.C;  // the 36-plane contraction, as ops 12 would run it
            n.bytes = 4.0 * ((double)x.C * x.H * x.W + 36.0 * x.C * OC + (double)OC * OH * OW);
            n.kern = wg4_conv_kernel_name(x.C, x.H, x.W, OC);
        }
    } else if (K == 3 && s == 1 && p == 1 && pad_end == 0 && (add_mode == 0 || add_mode == 2)) {
        // Winograd F(4,3): pad fused into op 15, madd (op 12), output + bias + act (op 11) (:425-463);
        // add_mode 2 adds `add` after the activation in op 11
        const int TW = (OW + 3) / 4, TH = (OH + 3) / 4, T = TW * TH;
        // plane rows padded to a multiple of 4 tiles: the madd GEMM then reads
        // whole float4s (and may copy them straight to LDS) on every tile
        const int ldt = (T + 3) & ~3;
        Scratch *sc = &sc_[lane_];
        sc->wg_need = std::max(sc->wg_need, (int64_t)36 * std::max(x.C, OC) * ldt);
        // The 36-plane intermediates dt / yt are shared by every Winograd
        // conv and allocated once the largest is known, so the launches
        // read their address at run time.  The workspace query only reads
        // shapes: a host sentinel stands in for their address there.
        const Img xi = x;
        const float *wg4 = W(name + ".wg4");
        const auto p_in = op_params(PPDL_OP_WG4_INPUT_PAD, T, TH), p_md = op_params(PPDL_OP_WG4_MADD, 0, 0),
                   p_out = op_params(PPDL_OP_WG4_OUTPUT, act, TW);
        const char *ech = getenv("PPDL_WG_CHAIN");
        const bool chaining = ech && ech[0] == '1';
        const ppdl_tview qd = planes(kShapeOnly, T, OC, ldt);
        const ppdl_tview qs[2] = {planes(kShapeOnly, T, x.C, ldt), view(wg4, {OC, x.C, 36})};
        const int64_t wsb = ppdl_hip_workspace_bytes(p_md.data(), &qd, qs, 2);
        if (wsb < 0 && bad_node_.empty()) bad_node_ = name;
        sc->ws_need = std::max(sc->ws_need, wsb);
        if (pend_.on && pend_.sc == sc && pend_.add_mode == 0 && pend_.y.d == x.d && pend_.y.C == x.C &&
            pend_.y.H == x.H && pend_.y.W == x.W && !x.ld && pend_.ldt == ldt && wg4_chain_fits(x.W)) {
            // the previous conv's output transform and this one's input transform
            const PendOut pp = pend_;
            pend_.on = false;
            node(pp.name + ".wg_chain", 1, [=](hipStream_t st) {
                return ok(wg4_chain(sc->yt, pp.bias, pp.y.d, sc->dt, xi.C, xi.W, xi.H, pp.act, ldt, ldt, st));
            });
        } else {
            node(name + ".wg_in", 1, [=](hipStream_t st) {
                ppdl_tview d = planes(sc->dt, T, xi.C, ldt), sx = view(xi);
                return ppdl_hip_run(p_in.data(), &d, &sx, 1, st);
            });
        }
        node(name + ".wg_madd", wsb > 0 ? 2 : 1, [=](hipStream_t st) {
            ppdl_tview d = planes(sc->yt, T, OC, ldt);
            std::vector<ppdl_tview> sv = {planes(sc->dt, T, xi.C, ldt), view(wg4, {OC, xi.C, 36})};
            if (wsb > 0) sv.push_back(view(sc->ws, {(sc->ws_bytes + 3) / 4}));
            return ppdl_hip_run(p_md.data(), &d, sv.data(), (int)sv.size(), st);
        });
        {
            GemmArgs g;
            bool im2col;
            if (gemm_args_of(p_md.data(), &qd, qs, &g, &im2col)) gemm_meta(1, g, wsb, im2col);
        }
        PendOut po;
        po.on = true;
        po.name = name;
        po.y = y;
        po.bias = b;
        po.add = add;
        po.act = act;
        po.add_mode = add_mode;
        po.ldt = ldt;
        po.TW = TW;
        po.TH = TH;
        po.sc = sc;
        po.p_out = p_out;
        pend_ = po;
        if (!chaining) flush_pending();
    } else {
        // k2, k3 s2: implicit-im2col GEMM + bias + act (op 16), replacing
        // im2col + mul_mat + permute/cont + add + act (:535-542)
        tagged(name, PPDL_OP_CONV_IM2COL, K | (s << 8) | (p << 16) | (act << 24), pad_end, view(y),
               {view(x), view(W(name + ".wr"), {OC, x.C, K * K}), vb});
    }
    return y;
}

// lin (:545-548): y = x W^T + b as a row-major-activation GEMM; optional act
// and fused add (residual) in the epilogue, and an optional prologue add
// (x + a_add, same layout as x) for output columns < a_add_n.
Seq Net::lin(const Seq &x, const std::string &name, int act, float *out, const float *add, int add_mode,
             const float *a_add, int a_add_n, const std::string &ln, float *ln_out) {
    const auto &ne = shape(name + ".weight");  // (in, out)
    const int in = (int)ne[0], nout = (int)ne[1];
    if (in != x.D && bad_node_.empty()) bad_node_ = name + " (feature mismatch)";
    Seq y{out ? out : alloc((int64_t)x.T * nout), x.T, nout, nout};
    GemmArgs g{};
    g.A = x.d;
    g.lda = x.ld;
    g.a_rowmajor = 1;
    g.B = W(name + ".wt");
    g.ldb = nout;
    g.C = y.d;
    g.ldc = nout;
    g.bias = W(name + ".bias");
    g.bias_n = 1;
    g.M = x.T;
    g.N = nout;
    g.K = in;
    g.batch = 1;
    g.act = act;
    g.add = add;
    g.add_mode = add_mode;
    g.a_add = a_add;
    g.a_add_n = a_add_n;
    if (!ln.empty()) {
        g.ln_g = W(ln + ".weight");
        g.ln_b = W(ln + ".bias");
        g.ln_out = ln_out;
    }
    gemm(name, g);
    return y;
}

// ln (:550-554): LN(a + b) * w + bias
Seq Net::ln(const Seq &a, const float *b, const std::string &name, float *out, int out_chw) {
    Seq y{out ? out : alloc((int64_t)a.T * kDM), a.T, kDM, kDM};
    const float *gm = W(name + ".weight"), *bt = W(name + ".bias");
    const Seq ai = a;
    node(name, 1, [=](hipStream_t st) { return ok(layernorm(ai.d, b, gm, bt, y.d, ai.T, out_chw, st)); });
    return y;
}

// second(relu(first(x))) for a 4-column x (the query-position MLP,
// :824-826) as one GEMM: the 4-in ReLU layer is computed in the second
// layer's A-operand loader, so its 300 x 512 hidden rows never reach memory
// With box_h: x is the previous layer's reference boxes and the GEMM first
// applies that layer's last box-head linear (bbox_head.2 on box_h) and the
// refinement to them in its loader, storing the refined boxes to box_out.
Seq Net::lin_in4(const Seq &x, const std::string &first, const std::string &second, int act, const Seq *box_h,
                 float *box_out) {
    const auto &n0 = shape(first + ".weight");   // (4, hidden)
    const auto &n1 = shape(second + ".weight");  // (hidden, out)
    if ((x.D != 4 || n0[0] != 4 || n1[0] != n0[1]) && bad_node_.empty()) bad_node_ = second + " (feature mismatch)";
    const int hid = (int)n0[1], nout = (int)n1[1];
    Seq y{alloc((int64_t)x.T * nout), x.T, nout, nout};
    GemmArgs g{};
    g.A = x.d;
    g.lda = x.ld;
    g.a_rowmajor = 1;
    g.a_w4 = W(first + ".wt");
    g.a_b4 = W(first + ".bias");
    g.B = W(second + ".wt");
    g.ldb = nout;
    g.C = y.d;
    g.ldc = nout;
    g.bias = W(second + ".bias");
    g.bias_n = 1;
    g.M = x.T;
    g.N = nout;
    g.K = hid;
    g.batch = 1;
    g.act = act;
    if (box_h) {
        const auto &nb = shape("bbox_head.2.weight");  // (256, 4)
        if ((nb[0] != box_h->D || nb[1] != 4) && bad_node_.empty()) bad_node_ = "bbox_head.2 (feature mismatch)";
        g.box_h = box_h->d;
        g.box_ldh = box_h->ld;
        g.box_k = box_h->D;
        g.box_w = W("bbox_head.2.wt");
        g.box_b = W("bbox_head.2.bias");
        g.box_out = box_out;
    }
    gemm(second, g);
    return y;
}

Seq Net::mlp3(const Seq &x, const std::string &pfx) {
    Seq h = lin(x, pfx + ".0", kActRelu);
    h = lin(h, pfx + ".1", kActRelu);
    return lin(h, pfx + ".2", kActNone);
}

// mha (:572-587) + output projection: q, k from x + pos, v from x, as one
// GEMM [T][768] = q | k | v whose prologue adds pos for the q|k columns;
// out = resid + o(attn) when resid given
Seq Net::mha(const Seq &x, const float *pos, const std::string &pfx, float *out, const float *resid) {
    const int T = x.T;
    Seq qkv = lin(x, pfx + ".qkv", kActNone, nullptr, nullptr, 0, pos, 2 * kDM);
    Seq att{alloc((int64_t)T * kDM), T, kDM, kDM};
    node(pfx + ".attn", 1, [=](hipStream_t st) {
        return ok(attention(qkv.d, 3 * kDM, qkv.d + kDM, 3 * kDM, qkv.d + 2 * kDM, 3 * kDM, att.d, kDM, T, st));
    });
    return lin(att, pfx + ".o", kActNone, out, resid, resid ? 2 : 0);
}

// hg_block (:598-614).  `cat` already holds the block input in its first
// `cin` channels; each layer writes its output into the next slice.
void Net::hg_block(const Img &cat, int cin, const std::string &pfx, bool light, int mid, Img *y, float *out,
                   const float *resid) {
    // a plane-strided concat (light blocks only) keeps its stride through the
    // layers' slots and the aggregation's middle map
    Img cur{cat.d, cin, cat.H, cat.W, cat.ld};
    const int64_t plane = cat.plane();
    for (int l = 0; l < 6; l++) {
        const std::string lp = pfx + ".l" + std::to_string(l);
        float *slot = cat.d + (cin + (int64_t)l * mid) * plane;
        if (light) {
            Img t = conv(cur, lp + ".c1", 1, 0, kActNone);
            cur = conv(t, lp + ".c2", 1, 2, kActRelu, slot, 0, nullptr, 0, cat.ld);  // depthwise k5 p2
        } else {
            cur = conv(cur, lp, 1, 1, kActRelu, slot);  // k3 p1
        }
    }
    Img full{cat.d, cin + 6 * mid, cat.H, cat.W, cat.ld};
    Img a = conv(full, pfx + ".agg0", 1, 0, kActRelu, nullptr, 0, nullptr, 0, cat.ld);
    *y = conv(a, pfx + ".agg1", 1, 0, kActRelu, out, 0, resid, resid ? 2 : 0);
}

// csp (:662-668): a = c1(x); 3x repvgg; b = c2(x); a + b.  repvgg (:656-660)
// = silu(c1_3x3(a) + c2_1x1(a)); the sums ride in the 1x1 convs' epilogues.
Img Net::csp(const Img &x, const std::string &pfx, float *out) {
    // PPDL_REPVGG=0 keeps the two-conv form of the RepVGG blocks (A/B runs)
    const char *e = getenv("PPDL_REPVGG");
    const bool fold = !(e && e[0] == '0');
    // c1 and c2 read the same input: one GEMM into [a | t2] (2C planes);
    // the last folded block adds t2 = silu(c2(x)) after its activation in
    // its output transform (PPDL_CSP_MERGE=0: two GEMMs, for A/B runs)
    const char *em = getenv("PPDL_CSP_MERGE");
    bool merge = fold && !(em && em[0] == '0') && w_.count(pfx + ".c12.wr");
    for (int i = 0; merge && i < 3; i++) merge = w_.count(pfx + ".bn" + std::to_string(i) + ".rep.wg4") > 0;
    if (merge) {
        const Img at = conv(x, pfx + ".c12", 1, 0, kActSilu);
        const int C = at.C / 2;
        Img a{at.d, C, at.H, at.W};
        const float *t2 = at.d + (int64_t)C * at.H * at.W;
        for (int i = 0; i < 3; i++) {
            const std::string bp = pfx + ".bn" + std::to_string(i);
            a = i < 2 ? conv(a, bp + ".rep", 1, 1, kActSilu) : conv(a, bp + ".rep", 1, 1, kActSilu, out, 0, t2, 2);
        }
        return a;
    }
    Img a = conv(x, pfx + ".c1", 1, 0, kActSilu);
    for (int i = 0; i < 3; i++) {
        const std::string bp = pfx + ".bn" + std::to_string(i);
        if (fold && w_.count(bp + ".rep.wg4")) {
            a = conv(a, bp + ".rep", 1, 1, kActSilu);  // silu(3x3 with the 1x1 folded into its centre tap)
        } else {
            Img t = conv(a, bp + ".c1", 1, 1, kActNone);
            a = conv(a, bp + ".c2", 1, 0, kActSilu, nullptr, 0, t.d, 1);
        }
    }
    return conv(x, pfx + ".c2", 1, 0, kActSilu, out, 0, a.d, 2);
}

// ---------------------------------------------------------------------------
// The full graph (builder::build, src/ppdoclayout.cpp:733-882).
bool Net::build(bool dumps, std::string *err) {
    want_dumps_ = dumps;
    for (int l = 0; l < kLanes; l++) {
        if (hipStreamCreateWithFlags(&lanes_[l], hipStreamNonBlocking) != hipSuccess) {
            *err = "hipStreamCreate failed";
            return false;
        }
    }
    stream_ = lanes_[0];  // the main lane; destroyed as stream_
    if (const char *e = getenv("PPDL_GRAPH_LANES")) multi_lane_ = e[0] == '1';
    image_ = alloc(3LL * IMG * IMG);
    pos_ = alloc(625LL * kDM);
    valid_ = alloc(NTOK);

    // ---- backbone (:616-652)
    Img img{image_, 3, IMG, IMG};
    Img x = conv(img, "stem1", 2, 1, kActRelu);  // 400, 32
    dump("stem1", x);
    Img cat0{alloc(64LL * 400 * 400), 64, 400, 400};  // [maxpool(xp) | stem2b]
    {
        const Img xi = x;
        node("stem.pool", 1, [=](hipStream_t st) { return ok(maxpool2_padend(xi.d, cat0.d, 32, 400, 400, st)); });
    }
    Img a = conv(x, "stem2a", 1, 0, kActRelu, nullptr, 1);        // pad(1,1) then k2 -> 400, 16
    conv(a, "stem2b", 1, 0, kActRelu, cat0.d + 32LL * 400 * 400, 1);  // -> 400, 32
    x = conv(cat0, "stem3", 2, 1, kActRelu);                        // 200, 32
    Img cat_s0{alloc((48 + 6 * 48LL) * 200 * 200), 48 + 6 * 48, 200, 200};
    x = conv(x, "stem4", 1, 0, kActRelu, cat_s0.d);  // 200, 48
    dump("stem", x);

    Img s0, s1, s2, s3;
    hg_block(cat_s0, 48, "st0.b0", false, 48, &s0, nullptr, nullptr);  // 200, 128
    dump("st0", s0);
    Img cat_s1{alloc((128 + 6 * 96LL) * 100 * 100), 128 + 6 * 96, 100, 100};
    conv(s0, "st1.ds", 2, 1, kActNone, cat_s1.d);  // dw -> 100, 128
    hg_block(cat_s1, 128, "st1.b0", false, 96, &s1, nullptr, nullptr);  // 100, 512
    dump("st1", s1);
    const int64_t p50 = 50 * 50;
    Img cat_b0{alloc((512 + 6 * 192LL) * p50), 512 + 6 * 192, 50, 50};
    Img cat_b1{alloc((1024 + 6 * 192LL) * p50), 1024 + 6 * 192, 50, 50};
    Img cat_b2{alloc((1024 + 6 * 192LL) * p50), 1024 + 6 * 192, 50, 50};
    conv(s1, "st2.ds", 2, 1, kActNone, cat_b0.d);  // dw -> 50, 512
    Img t;
    hg_block(cat_b0, 512, "st2.b0", true, 192, &t, cat_b1.d, nullptr);         // -> b1 input
    hg_block(cat_b1, 1024, "st2.b1", true, 192, &t, cat_b2.d, cat_b1.d);       // + residual
    hg_block(cat_b2, 1024, "st2.b2", true, 192, &s2, nullptr, cat_b2.d);       // + residual
    dump("st2", s2);
    // The 25x25 maps of stage 3 keep a 628-float plane stride (625 rounded
    // up to whole float4s), so the aggregation GEMMs' B rows are 16-byte
    // aligned and take the direct-to-LDS loader.
    const int64_t ld25 = 628;
    Img cat_s3{alloc((1024 + 6 * 384LL) * ld25), 1024 + 6 * 384, 25, 25, ld25};
    conv(s2, "st3.ds", 2, 1, kActNone, cat_s3.d, 0, nullptr, 0, ld25);  // dw -> 25, 1024
    hg_block(cat_s3, 1024, "st3.b0", true, 384, &s3, nullptr, nullptr);  // 25, 2048
    dump("st3", s3);

    // ---- hybrid encoder (:674-729)
    Img cat8{alloc(512LL * 10000), 512, 100, 100}, cat16{alloc(512LL * 2500), 512, 50, 50};
    Img catp16{alloc(512LL * 2500), 512, 50, 50}, catp32{alloc(512LL * 625), 512, 25, 25};
    conv(s1, "enc_in0", 1, 0, kActNone, cat8.d + 256LL * 10000);  // p8 -> fpn1 concat slice 1
    conv(s2, "enc_in1", 1, 0, kActNone, cat16.d + 256LL * 2500);  // p16 -> fpn0 concat slice 1
    Img p32 = conv(s3, "enc_in2", 1, 0, kActNone);                 // 25, 256
    {
        // AIFI (:683-696): to_seq, q = k = s + pos (in the q|k|v GEMM), post-norm MHA and FFN
        Seq s{alloc(625LL * kDM), 625, kDM, kDM};
        const Img pi = p32;
        node("aifi.to_seq", 1, [=](hipStream_t st) { return ok(transpose(pi.d, s.d, kDM, 625, kDM, st)); });
        Seq at = mha(s, pos_, "aifi", nullptr, nullptr);
        Seq s1n = ln(at, s.d, "aifi.ln1");
        Seq ff = lin(lin(s1n, "aifi.fc1", kActGelu), "aifi.fc2", kActNone);
        Seq back = ln(ff, s1n.d, "aifi.ln2", nullptr, 1);  // channel-major == (25,25,256) image
        p32.d = back.d;
    }
    dump("aifi", p32);
    Img lat0 = conv(p32, "lat0", 1, 0, kActSilu, catp32.d + 256LL * 625);  // also pan1's concat slice 1
    node("up0", 1, [=](hipStream_t st) { return ok(interp(lat0.d, nullptr, cat16.d, 256, 25, 25, 50, 50, 0, st)); });
    Img f16 = csp(cat16, "fpn0", nullptr);
    Img lat1 = conv(f16, "lat1", 1, 0, kActSilu, catp16.d + 256LL * 2500);  // also pan0's concat slice 1
    node("up1", 1, [=](hipStream_t st) { return ok(interp(lat1.d, nullptr, cat8.d, 256, 50, 50, 100, 100, 0, st)); });
    Img f8 = csp(cat8, "fpn1", nullptr);
    dump("f8", f8);
    conv(f8, "pand0", 2, 1, kActSilu, catp16.d);
    Img n16 = csp(catp16, "pan0", nullptr);
    dump("n16", n16);
    conv(n16, "pand1", 2, 1, kActSilu, catp32.d);
    Img n32 = csp(catp32, "pan1", nullptr);
    dump("n32", n32);

    // mask feature head (:711-724), on lane 1: only the encoder masks (after
    // the top-300 selection) and the final masks read it
    fork(1);
    Img h0 = conv(f8, "mh0.0", 1, 1, kActSilu);  // 100, 64
    Img h1 = conv(n16, "mh1.0", 1, 1, kActSilu);
    Img m1{alloc(64LL * 10000), 64, 100, 100};
    node("mh1.up", 1, [=](hipStream_t st) { return ok(interp(h1.d, h0.d, m1.d, 64, 50, 50, 100, 100, 1, st)); });
    Img h2 = conv(n32, "mh2.0", 1, 1, kActSilu);
    Img h2u{alloc(64LL * 2500), 64, 50, 50};
    node("mh2.up", 1, [=](hipStream_t st) { return ok(interp(h2.d, nullptr, h2u.d, 64, 25, 25, 50, 50, 1, st)); });
    Img h2b = conv(h2u, "mh2.2", 1, 1, kActSilu);
    Img mf{alloc(64LL * 10000), 64, 100, 100};
    node("mh2.up2", 1, [=](hipStream_t st) { return ok(interp(h2b.d, m1.d, mf.d, 64, 50, 50, 100, 100, 1, st)); });
    Img mo = conv(mf, "mh.out", 1, 1, kActSilu);
    Img ml = conv(s0, "mlat", 1, 1, kActSilu);  // 200, 64
    Img mu{alloc(64LL * 40000), 64, 200, 200};
    node("mh.up", 1, [=](hipStream_t st) { return ok(interp(mo.d, ml.d, mu.d, 64, 100, 100, 200, 200, 1, st)); });
    Img mb = conv(mu, "mout.base", 1, 1, kActSilu);
    Img mask_feat = conv(mb, "mout.conv", 1, 0, kActNone);  // 200, 32
    dump("mask_feat", mask_feat);
    main_lane();

    // ---- decoder inputs (:791-801): 1x1 projections written channel-major
    // into one (256, LDT) sourceT, level after level along the token axis.
    // Channel-major makes sourceT the k-major A operand of the value and
    // enc_out projections, whose GEMMs then run on the DMA-staged kernel (a
    // row-major A has no DMA loader); the tokens are padded to LDT = 13128
    // so that M and the leading dimension are multiples of 4.  The padding
    // columns hold no data: the GEMMs compute rows 13125..13127 from them and
    // nothing reads those rows.  PPDL_SOURCE_TM=1 keeps the token-major
    // source and the row-major GEMMs (A/B runs, tests).
    const char *etm = getenv("PPDL_SOURCE_TM");
    const bool src_tm = etm && etm[0] == '1';
    constexpr int LDT = (NTOK + 3) / 4 * 4;
    float *sbuf = alloc((int64_t)LDT * kDM);
    {
        const Img lv[3] = {f8, n16, n32};
        const int start[3] = {0, 10000, 12500};
        for (int l = 0; l < 3; l++) {
            const std::string nm = "dec_in" + std::to_string(l);
            const int P = lv[l].H * lv[l].W;
            GemmArgs g{};
            g.A = W(nm + ".wr");
            g.lda = kDM;
            g.B = lv[l].d;
            g.ldb = P;
            g.C = src_tm ? sbuf + (int64_t)start[l] * kDM : sbuf + start[l];
            g.ldc = src_tm ? kDM : LDT;
            g.c_trans = src_tm ? 1 : 0;
            g.bias = W(nm + ".bias");
            g.M = kDM;
            g.N = P;
            g.K = lv[l].C;
            g.batch = 1;
            gemm(nm, g, 1);  // a 1x1 conv (src/ppdoclayout.cpp:786-788)
        }
    }
    // the linear `name` of a source-shaped x (either layout); y has LDT rows
    const auto lin_src = [&](const float *x, const std::string &name, float *out) {
        if (src_tm) return lin(Seq{const_cast<float *>(x), NTOK, kDM, kDM}, name, kActNone, out);
        const auto &ne = shape(name + ".weight");  // (in, out)
        const int nout = (int)ne[1];
        if ((int)ne[0] != kDM && bad_node_.empty()) bad_node_ = name + " (feature mismatch)";
        Seq y{out ? out : alloc((int64_t)LDT * nout), NTOK, nout, nout};
        GemmArgs g{};
        g.A = x;  // k-major: A[k][m] = x[k * LDT + m]
        g.lda = LDT;
        g.B = W(name + ".wt");
        g.ldb = nout;
        g.C = y.d;
        g.ldc = nout;
        g.bias = W(name + ".bias");
        g.bias_n = 1;
        g.M = LDT;
        g.N = nout;
        g.K = kDM;
        g.batch = 1;
        gemm(name, g);
        return y;
    };
    if (want_dumps_) {
        if (src_tm) {
            dump("source", sbuf, {kDM, NTOK});
        } else {
            float *tm = alloc((int64_t)LDT * kDM);
            node("source.tm", 1, [=](hipStream_t st) { return ok(transpose(sbuf, tm, kDM, LDT, kDM, st)); });
            dump("source", tm, {kDM, NTOK});
        }
    }
    // value projections of all six decoder layers at once (layer i: columns
    // 256i..256i+255), on lane 2 until the first deformable attention
    fork(2);
    const Seq vcat = lin_src(sbuf, "dec.ca.vp", nullptr);
    main_lane();
    // memory = source * valid (:797), consumed only by enc_out.l.  valid is 0
    // or 1 per token, so enc_out.l(memory) equals enc_out.l(source) on valid
    // rows and the bias row on masked ones (a zero row through the GEMM: every
    // product is a zero, as long as source is finite): the GEMM runs on
    // source and the LayerNorm takes the bias for masked rows.  PPDL_MEMORY=1
    // keeps the multiply as its own node (channel-major source: through a
    // token-major copy and back, both exact).
    const char *emem = getenv("PPDL_MEMORY");
    Seq om;
    if (emem && emem[0] == '1') {
        float *mem = alloc((int64_t)LDT * kDM);
        if (src_tm) {
            node("memory", 1, [=](hipStream_t st) { return ok(mul_rows(sbuf, valid_, mem, NTOK, kDM, st)); });
        } else {
            float *tm = alloc((int64_t)LDT * kDM), *mt = alloc((int64_t)LDT * kDM);
            node("memory", 3, [=](hipStream_t st) {
                hipError_t e = transpose(sbuf, tm, kDM, LDT, kDM, st);
                if (e == hipSuccess) e = mul_rows(tm, valid_, mt, NTOK, kDM, st);
                if (e == hipSuccess) e = transpose(mt, mem, LDT, kDM, LDT, st);
                return ok(e);
            });
        }
        om = ln(lin_src(mem, "enc_out.l", nullptr), nullptr, "enc_out.ln");
    } else {
        const Seq eo = lin_src(sbuf, "enc_out.l", nullptr);
        om = Seq{alloc((int64_t)NTOK * kDM), NTOK, kDM, kDM};
        const float *gm = W("enc_out.ln.weight"), *bt = W("enc_out.ln.bias"), *fill = W("enc_out.l.bias");
        const float *mask = valid_;
        const Seq o = om;
        node("enc_out.ln", 1, [=](hipStream_t st) {
            return ok(layernorm(eo.d, nullptr, gm, bt, o.d, NTOK, 0, st, mask, fill));
        });
    }
    Seq ecls = lin(om, "score_head", kActNone);  // (13125, 25)
    topk_ = (int32_t *)alloc(NQ);
    tagged("topk300", PPDL_OP_TOPK, 0, 0, view(topk_, {NQ}, PPDL_TYPE_I32), {view(ecls.d, {NC, NTOK})});
    dump("topk_idx", topk_, {NQ}, true);
    Seq target{alloc((int64_t)NQ * kDM), NQ, kDM, kDM};
    node("target", 1, [=](hipStream_t st) { return ok(get_rows(om.d, topk_, target.d, NQ, st)); });
    dump("target", target.d, {kDM, NQ});

    // enhanced reference from the encoder masks (:808-822)
    // mask logits = mask queries x prototypes.  Inference only needs their
    // signs (the box of each encoder mask, the final binary masks), so the
    // graph's GEMMs store sign bits from the epilogue (1.5 MB instead of
    // 48 MB each); the logits themselves are computed in dump mode and on
    // request (ppdl_get_raw) by the same GEMM without the bits.
    auto masks_args = [&](const Seq &mq, float *out, uint32_t *bits) {
        GemmArgs g{};
        g.A = mq.d;
        g.lda = mq.ld;
        g.a_rowmajor = 1;
        g.B = mask_feat.d;
        g.ldb = NPIX;
        g.C = out;
        g.ldc = NPIX;
        g.M = NQ;
        g.N = NPIX;
        g.K = 32;
        g.batch = 1;
        g.bits = bits;
        return g;
    };
    Seq outq0 = ln(target, nullptr, "dec_norm");
    Seq mq0 = mlp3(outq0, "mq");
    uint32_t *encbits = (uint32_t *)alloc((int64_t)NQ * (NPIX / 32));
    join(1);
    gemm("enc_masks", masks_args(mq0, nullptr, encbits));
    if (want_dumps_) {
        float *encm = alloc((int64_t)NQ * NPIX);
        gemm("enc_masks.logits", masks_args(mq0, encm, nullptr));
        dump("enc_masks", encm, {NPIX, NQ});
    }
    refu_ = alloc((int64_t)NQ * 4);
    node("mask_box", 1, [=](hipStream_t st) { return ok(mask_box_bits(encbits, refu_, NQ, st)); });
    dump("init_ref_unact", refu_, {4, NQ});
    boxes_ = alloc((int64_t)NQ * 4);
    node("ref0", 1, [=](hipStream_t st) {
        hipError_t e = hipMemcpyAsync(boxes_, refu_, NQ * 4 * sizeof(float), hipMemcpyDeviceToDevice, st);
        return e == hipSuccess ? ok(box_update(nullptr, boxes_, NQ * 4, st)) : 3;
    });

    // ---- decoder layers (:824-863)
    Seq ref{boxes_, NQ, 4, 4};
    Seq xq = target;
    const char *dln = getenv("PPDL_DEC_LN");
    const bool fused_ln = !(dln && dln[0] == '0');
    // Layers 1-5 refine the boxes of the previous layer inside their
    // query-position GEMM (bbox_head.2 + refinement in its loader, the
    // refined boxes stored to a buffer of their own); the last layer's
    // bbox_head.2 writes the result boxes.  PPDL_BOX_FUSE=0: every layer's
    // bbox_head.2 refines boxes_ in place.
    const char *ebf = getenv("PPDL_BOX_FUSE");
    const bool box_fuse = !(ebf && ebf[0] == '0');
    Seq bh_prev;
    for (int i = 0; i < 6; i++) {
        const std::string dp = "dec" + std::to_string(i);
        Seq qpos;
        if (box_fuse && i > 0) {
            float *ref_new = alloc((int64_t)NQ * 4);
            qpos = lin_in4(ref, "qpos.0", "qpos.1", kActNone, &bh_prev, ref_new);
            ref = Seq{ref_new, NQ, 4, 4};
        } else {
            qpos = lin_in4(ref, "qpos.0", "qpos.1", kActNone);
        }
        // The post-residual layer norms (ln1..ln3) run in the A loader of the
        // GEMM that consumes them, which also stores the normed rows for
        // the residual add two GEMMs later: no layer-norm launches
        // (PPDL_DEC_LN=0: separate layer-norm launches, for A/B runs).
        // lnz(z, norm, out): out = norm(z) as its own launch, or nothing
        // here and the norm's name for the consumer's loader.
        auto lnz = [&](const Seq &z, const std::string &norm, Seq &out) -> std::string {
            if (!fused_ln) {
                ln(z, nullptr, norm, out.d);
                return "";
            }
            return norm;
        };
        Seq sa = mha(xq, qpos.d, dp + ".sa", nullptr, xq.d);  // z1 = x + attn, q = k = x + qpos
        Seq x1{alloc((int64_t)NQ * kDM), NQ, kDM, kDM};       // ln1(z1)
        const std::string n1 = lnz(sa, dp + ".ln1", x1);
        if (i == 0) join(2);
        // sampling offsets | attention logits of (ln1(z1) + qpos), one [NQ][288] GEMM
        Seq soaw = lin(fused_ln ? sa : x1, dp + ".ca.soaw", kActNone, nullptr, nullptr, 0, qpos.d, 1 << 30, n1, x1.d);
        Seq ca{alloc((int64_t)NQ * kDM), NQ, kDM, kDM};
        tagged(dp + ".msdeform", PPDL_OP_MSDEF, 0, 0, view(ca.d, {kDM, NQ}),
               {row_view(vcat.d + (int64_t)i * kDM, kDM, NTOK, vcat.ld), row_view(soaw.d, 192, NQ, soaw.ld),
                row_view(soaw.d + 192, 96, NQ, soaw.ld), view(ref.d, {4, NQ})});
        Seq cao = lin(ca, dp + ".ca.op", kActNone, nullptr, x1.d, 2);  // z2 = x1 + ca
        Seq x2{alloc((int64_t)NQ * kDM), NQ, kDM, kDM};                // ln2(z2)
        const std::string n2 = lnz(cao, dp + ".ln2", x2);
        Seq h1 = lin(fused_ln ? cao : x2, dp + ".fc1", kActRelu, nullptr, nullptr, 0, nullptr, 0, n2, x2.d);
        Seq ff = lin(h1, dp + ".fc2", kActNone, nullptr, x2.d, 2);  // z3 = x2 + ffn
        Seq x3{alloc((int64_t)NQ * kDM), NQ, kDM, kDM};             // ln3(z3): the layer's output
        const std::string n3 = lnz(ff, dp + ".ln3", x3);
        // box refinement ref = sigmoid(delta + inv_sigmoid(ref)) in the last
        // bbox-head GEMM's epilogue, in place
        Seq bh0 = lin(fused_ln ? ff : x3, "bbox_head.0", kActRelu, nullptr, nullptr, 0, nullptr, 0, n3, x3.d);
        xq = x3;
        static const char *hn[6] = {"hidden0", "hidden1", "hidden2", "hidden3", "hidden4", "hidden5"};
        dump(hn[i], xq.d, {kDM, NQ});
        Seq bh = lin(bh0, "bbox_head.1", kActRelu);
        if (box_fuse && i < 5) bh_prev = bh;
        else lin(bh, "bbox_head.2", kActNone, boxes_, ref.d, 3);  // boxes_ = refine(delta, ref)
    }

    // ---- heads (:865-876)
    Seq outq = ln(xq, nullptr, "dec_norm");
    Seq lg = lin(outq, "score_head", kActNone);
    logits_ = lg.d;
    Seq mq6 = mlp3(outq, "mq");
    masks_ = alloc((int64_t)NQ * NPIX);
    mbits_ = (uint32_t *)alloc((int64_t)NQ * (NPIX / 32));
    gemm("masks", masks_args(mq6, nullptr, mbits_));  // the result's binary masks
    mask_logits_ = masks_args(mq6, masks_, nullptr);
    Seq gp = lin(lin(xq, "order5", kActNone), "gp", kActNone);  // (300, 128)
    order_ = alloc((int64_t)NQ * NQ);
    node("order", 1, [=](hipStream_t st) { return ok(order_logits(gp.d, order_, NQ, 64, 1.0f / 8.0f, st)); });

    if (pend_.on) flush_pending();
    if (!missing_.empty()) {
        *err = "missing tensor: " + missing_;
        return false;
    }
    if (!bad_node_.empty()) {
        *err = "node rejected by the op contract: " + bad_node_;
        return false;
    }
    if (lane_ != 0 && bad_node_.empty()) bad_node_ = "unjoined lane";
    for (Scratch &sc : sc_) {
        sc.dt = sc.wg_need ? alloc(sc.wg_need) : nullptr;
        sc.yt = sc.wg_need ? alloc(sc.wg_need) : nullptr;
        sc.ws_bytes = (sc.ws_need + 255) / 256 * 256;
        sc.ws = sc.ws_bytes ? alloc(sc.ws_bytes / 4) : nullptr;
    }
    if (oom_) {
        *err = "device allocation failed while building the graph";
        return false;
    }

    // host constants (:887-923)
    std::vector<float> pos(625 * kDM), vm(NTOK);
    double omega[64];
    for (int i = 0; i < 64; i++) omega[i] = 1.0 / std::pow(10000.0, (double)i / 64.0);
    for (int hh = 0; hh < 25; hh++)
        for (int ww = 0; ww < 25; ww++) {
            float *pp = pos.data() + (size_t)(hh * 25 + ww) * kDM;
            for (int i = 0; i < 64; i++) {
                pp[i] = (float)std::sin(hh * omega[i]);
                pp[64 + i] = (float)std::cos(hh * omega[i]);
                pp[128 + i] = (float)std::sin(ww * omega[i]);
                pp[192 + i] = (float)std::cos(ww * omega[i]);
            }
        }
    {
        const int lw[3] = {100, 50, 25};
        const float eps = 1e-2f;
        int t2 = 0;
        for (int l = 0; l < 3; l++) {
            const float wh = 0.05f * (float)std::pow(2.0f, (float)l);
            for (int yy = 0; yy < lw[l]; yy++)
                for (int xx = 0; xx < lw[l]; xx++) {
                    const float cx = ((float)xx + 0.5f) / (float)lw[l], cy = ((float)yy + 0.5f) / (float)lw[l];
                    const bool okv = cx > eps && cx < 1.0f - eps && cy > eps && cy < 1.0f - eps && wh > eps &&
                                     wh < 1.0f - eps;
                    vm[t2++] = okv ? 1.0f : 0.0f;
                }
        }
    }
    if (hipMemcpy(pos_, pos.data(), pos.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(valid_, vm.data(), vm.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        *err = "upload of host constants failed";
        return false;
    }
    return true;
}

// One eager pass (every node validated and launched), then stream capture of
// the same sequence into a hipGraph.
bool Net::capture(std::string *err) {
    std::vector<float> zero(3LL * IMG * IMG, 0.0f);
    if (!upload_image(zero.data())) {
        *err = "image upload failed";
        return false;
    }
    if (const int rc = launch_all()) {
        *err = "eager pass failed at node " + failed_ + " (" + std::to_string(rc) + ")";
        return false;
    }
    if (hipStreamSynchronize(stream_) != hipSuccess) {
        *err = "eager pass failed";
        return false;
    }
    if (hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        *err = "hipStreamBeginCapture failed";
        return false;
    }
    const int rc = launch_all();
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(stream_, &g);
    if (rc || e != hipSuccess || !g) {
        if (g) (void)hipGraphDestroy(g);
        *err = "graph capture failed";
        return false;
    }
    graph_ = g;
    if (hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0) != hipSuccess) {
        *err = "hipGraphInstantiate failed";
        return false;
    }
    return true;
}

int Net::launch_all() {
    for (auto &n : nodes_) {
        int rc = 0;
        if (n.kind == 1)
            rc = (hipEventRecord(events_[n.ev], stream_) == hipSuccess &&
                  hipStreamWaitEvent(lanes_[n.lane], events_[n.ev], 0) == hipSuccess)
                     ? 0
                     : 3;
        else if (n.kind == 2)
            rc = (hipEventRecord(events_[n.ev], lanes_[n.lane]) == hipSuccess &&
                  hipStreamWaitEvent(stream_, events_[n.ev], 0) == hipSuccess)
                     ? 0
                     : 3;
        else
            rc = n.run(lanes_[n.lane]);
        if (rc) {
            failed_ = n.name;
            return rc;
        }
    }
    return 0;
}

bool Net::upload_image(const float *host) {
    return hipMemcpyAsync(image_, host, 3LL * IMG * IMG * 4, hipMemcpyHostToDevice, stream_) == hipSuccess &&
           hipStreamSynchronize(stream_) == hipSuccess;
}

bool Net::download(float *logits, float *boxes, float *order, uint32_t *mbits) {
    const hipStream_t s = stream_;
    return hipMemcpyAsync(logits, logits_, (size_t)NQ * NC * 4, hipMemcpyDeviceToHost, s) == hipSuccess &&
           hipMemcpyAsync(boxes, boxes_, (size_t)NQ * 4 * 4, hipMemcpyDeviceToHost, s) == hipSuccess &&
           hipMemcpyAsync(order, order_, (size_t)NQ * NQ * 4, hipMemcpyDeviceToHost, s) == hipSuccess &&
           hipMemcpyAsync(mbits, mbits_, (size_t)NQ * (NPIX / 32) * 4, hipMemcpyDeviceToHost, s) == hipSuccess &&
           hipStreamSynchronize(s) == hipSuccess;
}

bool Net::mask_logits() {
    return gemm_dense(mask_logits_, GemmWorkspace{nullptr, 0}, stream_) == hipSuccess &&
           hipStreamSynchronize(stream_) == hipSuccess;
}

int Net::replay() {
    if (hipGraphLaunch(exec_, stream_) != hipSuccess) return 2;
    return hipStreamSynchronize(stream_) == hipSuccess ? 0 : 2;
}

double Net::time_graph(int iters) {
    hipEvent_t e0, e1;
    if (iters < 1 || hipEventCreate(&e0) != hipSuccess) return -1.0;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return -1.0;
    }
    bool good = hipEventRecord(e0, stream_) == hipSuccess;
    for (int i = 0; good && i < iters; i++) good = hipGraphLaunch(exec_, stream_) == hipSuccess;
    good = good && hipEventRecord(e1, stream_) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
    float ms = 0.0f;
    good = good && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return good ? (double)ms / iters : -1.0;
}

// Per-node device time as the graph sees it: each node is captured `iters`
// times into a graph of its own, which is replayed once untimed and once
// between two HIP events on the graph's stream.  (Eager launches would add
// the host's per-launch cost, several µs, to every short kernel.)  Nodes that
// update a buffer in place drift its contents meanwhile; the next ppdl_infer /
// ppdl_compute recomputes everything from the image.
// In-graph mode (iters < 0): the whole node list captured once into one
// graph with a one-lane kernel storing the device wall clock in front of it
// and after every kernel node, replayed -iters times; a node's time is the
// mean interval between its stamp and the previous one, less the interval
// of two stamps with nothing between them: its share of a replay in context
// (operands as the previous nodes left them).  One stream only.
int Net::profile_in_graph(int reps, ppdl_node_stat *out, int cap) {
    if (multi_lane_ || reps < 1) return -1;
    std::vector<size_t> idx;
    for (size_t i = 0; i < nodes_.size(); i++)
        if (nodes_[i].kind == 0) idx.push_back(i);
    const size_t ns = idx.size() + 2;  // stamps: front, after each node, one more for the baseline
    unsigned long long *dstamp = nullptr;
    int khz = 0;
    bool good = hipMalloc((void **)&dstamp, ns * sizeof(unsigned long long)) == hipSuccess &&
                hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0) == hipSuccess && khz > 0;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    if (good) {
        good = hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) == hipSuccess;
        bool ran = good && stamp(dstamp, stream_) == hipSuccess;
        for (size_t k = 0; ran && k < idx.size(); k++)
            ran = nodes_[idx[k]].run(stream_) == 0 && stamp(dstamp + k + 1, stream_) == hipSuccess;
        ran = ran && stamp(dstamp + idx.size() + 1, stream_) == hipSuccess;
        good = good && hipStreamEndCapture(stream_, &g) == hipSuccess && ran;  // capture always ended
        good = good && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess;
    }
    std::vector<unsigned long long> h(ns);
    std::vector<double> acc(idx.size(), 0.0);
    double base = 0.0;
    good = good && hipGraphLaunch(ge, stream_) == hipSuccess && hipStreamSynchronize(stream_) == hipSuccess;
    for (int r = 0; good && r < reps; r++) {
        good = hipGraphLaunch(ge, stream_) == hipSuccess && hipStreamSynchronize(stream_) == hipSuccess &&
               hipMemcpy(h.data(), dstamp, ns * sizeof(unsigned long long), hipMemcpyDeviceToHost) == hipSuccess;
        for (size_t k = 0; good && k < idx.size(); k++) acc[k] += (double)(h[k + 1] - h[k]);
        base += (double)(h[ns - 1] - h[ns - 2]);
    }
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    if (dstamp) (void)hipFree(dstamp);
    if (!good) return -1;
    const double us_per_tick = 1000.0 / khz;
    base = base / reps * us_per_tick;
    int n = 0;
    for (size_t k = 0; k < idx.size() && n < cap; k++) {
        const Node &nd = nodes_[idx[k]];
        ppdl_node_stat &o = out[n++];
        memset(&o, 0, sizeof(o));
        snprintf(o.name, sizeof(o.name), "%s", nd.name.c_str());
        snprintf(o.kernel, sizeof(o.kernel), "%s", nd.kern.c_str());
        o.cls = nd.cls;
        o.kernels = nd.kernels;
        o.flops = nd.flops;
        o.bytes = nd.bytes;
        o.us = acc[k] / reps * us_per_tick - base;
    }
    return n;
}

int Net::profile_nodes(int iters, ppdl_node_stat *out, int cap) {
    if (iters < 0) return profile_in_graph(-iters, out, cap);
    hipEvent_t e0, e1;
    if (iters < 1 || hipEventCreate(&e0) != hipSuccess) return -1;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return -1;
    }
    int n = 0;
    bool good = true;
    for (size_t i = 0; good && i < nodes_.size() && n < cap; i++) {
        Node &nd = nodes_[i];
        if (nd.kind != 0) continue;
        hipGraph_t g = nullptr;
        hipGraphExec_t ge = nullptr;
        good = hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) == hipSuccess;
        bool ran = good;
        for (int r = 0; ran && r < iters; r++) ran = nd.run(stream_) == 0;
        good = good && hipStreamEndCapture(stream_, &g) == hipSuccess && ran;  // capture always ended
        good = good && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess;
        good = good && hipGraphLaunch(ge, stream_) == hipSuccess;
        good = good && hipEventRecord(e0, stream_) == hipSuccess && hipGraphLaunch(ge, stream_) == hipSuccess;
        good = good && hipEventRecord(e1, stream_) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
        float ms = 0.0f;
        good = good && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
        if (ge) (void)hipGraphExecDestroy(ge);
        if (g) (void)hipGraphDestroy(g);
        ppdl_node_stat &o = out[n++];
        memset(&o, 0, sizeof(o));
        snprintf(o.name, sizeof(o.name), "%s", nd.name.c_str());
        snprintf(o.kernel, sizeof(o.kernel), "%s", nd.kern.c_str());
        o.cls = nd.cls;
        o.kernels = nd.kernels;
        o.flops = nd.flops;
        o.bytes = nd.bytes;
        o.us = 1000.0 * ms / iters;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return good ? n : -1;
}

// ---------------------------------------------------------------------------
// Host result assembly: the reference's postprocess (src/ppdoclayout.cpp:
// 927-993) on this runtime's downloads.  The graph's mask GEMM stores the
// logits' sign bits, so 1.5 MB crosses PCIe instead of 48 MB.
// On the host:
//   * every (query, class) logit is scored with the logistic function, and
//     the 300 best are picked by a 64-bit key: the score's order-preserving
//     bits, then the complemented flat index (lower index first on ties);
//   * queries are placed in reading order by their pairwise-vote totals,
//     keyed by (vote, query index) ascending;
//   * the picked rows get label, score, the box restored to the original
//     size, the reading position, and their query's mask bits expanded.
// The float arithmetic (logistic as 1 / (1 + exp(-x)), each vote summed over
// i ascending, the box formulas) is the reference's, so results match it bit
// for bit.
struct HostOut {
    float *logits = nullptr, *boxes = nullptr, *order = nullptr;  // pinned downloads
    uint32_t *mbits = nullptr;
};

inline float logistic(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// uint32 whose unsigned order is the float order, with -0 taken as +0 (the
// two compare equal)
inline uint32_t sortable_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (u == 0x80000000u) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// pos[j] = reading position of query j.  R[i][j] = order[i * nq + j]; the
// vote of j sums logistic(R[i][j] - R[j][i]) over i != j in ascending i.
// Row i of R is streamed once and adds its term to every vote.
void reading_positions(const float *order, int nq, std::vector<int> &pos) {
    std::vector<float> vote((size_t)nq, 0.0f);
    for (int i = 0; i < nq; i++) {
        const float *ri = order + (size_t)i * nq;
        for (int j = 0; j < nq; j++)
            if (j != i) vote[(size_t)j] += logistic(ri[j] - order[(size_t)j * nq + i]);
    }
    std::vector<uint64_t> key((size_t)nq);
    for (int j = 0; j < nq; j++) key[(size_t)j] = ((uint64_t)sortable_bits(vote[(size_t)j]) << 32) | (uint32_t)j;
    std::sort(key.begin(), key.end());
    pos.assign((size_t)nq, 0);
    for (int r = 0; r < nq; r++) pos[(size_t)(uint32_t)key[(size_t)r]] = r;
}

// The k best of n scores, best first: higher score, then lower index.
void best_scores(const float *score, int n, int k, std::vector<int32_t> &pick) {
    std::vector<uint64_t> key((size_t)n);
    for (int f = 0; f < n; f++) key[(size_t)f] = ((uint64_t)sortable_bits(score[f]) << 32) | (uint32_t)~(uint32_t)f;
    std::nth_element(key.begin(), key.begin() + (k - 1), key.end(), std::greater<uint64_t>());
    std::sort(key.begin(), key.begin() + k, std::greater<uint64_t>());
    pick.resize((size_t)k);
    for (int r = 0; r < k; r++) pick[(size_t)r] = (int32_t)~(uint32_t)key[(size_t)r];
}

// out rows r = 0..rows-1 get the NPIX mask bits of query qrow[r] as int32
// 0/1, rows split over a few host threads
void expand_mask_bits(const uint32_t *bits, const std::vector<int> &qrow, int32_t *out) {
    constexpr int kWords = NPIX / 32;
    const int rows = (int)qrow.size();
    auto work = [&](int r0, int r1) {
        for (int r = r0; r < r1; r++) {
            const uint32_t *b = bits + (size_t)qrow[(size_t)r] * kWords;
            int32_t *o = out + (size_t)r * NPIX;
            for (int w = 0; w < kWords; w++, o += 32) {
                const uint32_t v = b[w];
                for (int t = 0; t < 32; t++) o[t] = (int32_t)((v >> t) & 1u);
            }
        }
    };
    const int nt = std::max(1, std::min<int>(8, (int)std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    const int per = (rows + nt - 1) / nt;
    for (int t = 1; t < nt && t * per < rows; t++) pool.emplace_back(work, t * per, std::min(rows, (t + 1) * per));
    work(0, std::min(rows, per));
    for (auto &th : pool) th.join();
}

void assemble_result(const HostOut &h, int ori_h, int ori_w, std::vector<float> &dets, std::vector<int32_t> &masks,
                     std::vector<int32_t> &pick) {
    std::vector<int> pos;
    reading_positions(h.order, NQ, pos);
    std::vector<float> score((size_t)NQ * NC);
    for (size_t f = 0; f < score.size(); f++) score[f] = logistic(h.logits[f]);
    best_scores(score.data(), NQ * NC, NQ, pick);
    // the original size the boxes are restored to (sf = 800 / ori, then
    // floor(800 / sf + 0.5))
    const float sf_h = (float)IMG / (float)ori_h, sf_w = (float)IMG / (float)ori_w;
    const float fh = std::floor((float)IMG / sf_h + 0.5f), fw = std::floor((float)IMG / sf_w + 0.5f);
    dets.resize((size_t)NQ * 7);
    std::vector<int> qrow((size_t)NQ);
    for (int r = 0; r < NQ; r++) {
        const int f = pick[(size_t)r], q = f / NC;
        qrow[(size_t)r] = q;
        const float cx = h.boxes[4 * q], cy = h.boxes[4 * q + 1], bw = h.boxes[4 * q + 2], bh = h.boxes[4 * q + 3];
        float *row = dets.data() + (size_t)r * 7;
        row[0] = (float)(f % NC);
        row[1] = score[(size_t)f];
        row[2] = (cx - bw * 0.5f) * fw;
        row[3] = (cy - bh * 0.5f) * fh;
        row[4] = (cx + bw * 0.5f) * fw;
        row[5] = (cy + bh * 0.5f) * fh;
        row[6] = (float)pos[(size_t)q];
    }
    masks.resize((size_t)NQ * NPIX);
    expand_mask_bits(h.mbits, qrow, masks.data());
}

bool write_file(const std::string &path, const void *src, size_t nbytes) {
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) return false;
    const size_t n = fwrite(src, 1, nbytes, f);
    fclose(f);
    return n == nbytes;
}

}  // namespace
}  // namespace ppdl

struct ppdl_ctx {
    std::unique_ptr<ppdl::Net> net;
    bool computed = false;  // a replay has run (dumps, ppdl_get_raw)
    bool fetched = false;   // `host` and the results belong to the last ppdl_infer
    ppdl::HostOut host;     // pinned download buffers
    void *pinned = nullptr;
    std::vector<float> dets;
    std::vector<int32_t> masks, picks;
    ~ppdl_ctx() {
        net.reset();
        if (pinned) (void)hipHostFree(pinned);
    }
    // one pinned block for the four downloads
    bool alloc_host() {
        using namespace ppdl;
        const size_t nl = (size_t)NQ * NC, nb = (size_t)NQ * 4, no = (size_t)NQ * NQ, nm = (size_t)NQ * (NPIX / 32);
        if (hipHostMalloc(&pinned, (nl + nb + no + nm) * 4, hipHostMallocDefault) != hipSuccess) {
            pinned = nullptr;
            return false;
        }
        float *f = (float *)pinned;
        host.logits = f;
        host.boxes = f + nl;
        host.order = f + nl + nb;
        host.mbits = (uint32_t *)(f + nl + nb + no);
        return true;
    }
};

extern "C" PPDL_API ppdl_ctx *ppdl_init_ex(const char *model_path, int backend, int enable_dumps) {
    if (!model_path) return nullptr;
    if (backend == PPDL_BACKEND_CPU) {
        fprintf(stderr, "ppdl: this build has no CPU backend; use PPDL_BACKEND_HIP\n");
        return nullptr;
    }
    if (backend != PPDL_BACKEND_CUDA && backend != PPDL_BACKEND_HIP) return nullptr;
    {
        // the file is checked before any device work, so a bad path or a
        // malformed file fails the same way on every host
        ppdl::GgufFile g;
        std::string err;
        if (!ppdl::gguf_open(model_path, &g, &err)) {
            fprintf(stderr, "ppdl: %s\n", err.c_str());
            return nullptr;
        }
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
        fprintf(stderr, "ppdl: no GPU backend available\n");
        return nullptr;
    }
    auto *c = new ppdl_ctx();
    c->net.reset(new ppdl::Net());
    std::string err;
    if (!c->net->load(model_path, &err) || !c->net->build(enable_dumps != 0, &err) || !c->net->capture(&err)) {
        fprintf(stderr, "ppdl: %s\n", err.c_str());
        delete c;
        return nullptr;
    }
    if (!c->alloc_host()) {
        err = "pinned host allocation failed";
        fprintf(stderr, "ppdl: %s\n", err.c_str());
        delete c;
        return nullptr;
    }
    fprintf(stderr, "ppdl: loaded %s; graph of %d kernel launches\n", model_path, c->net->nodes());
    return c;
}

extern "C" PPDL_API ppdl_ctx *ppdl_init(const char *model_path, int backend) {
    return ppdl_init_ex(model_path, backend, 0);
}

extern "C" PPDL_API int ppdl_compute(ppdl_ctx *c, const float *image_chw) {
    if (!c || !image_chw) return 1;
    if (!c->net->upload_image(image_chw)) return 2;
    const int rc = c->net->replay();
    if (rc == 0) c->computed = true;
    return rc;
}

extern "C" PPDL_API int ppdl_infer(ppdl_ctx *c, const float *image_chw, int ori_h, int ori_w, ppdl_result *res) {
    if (!c || !image_chw || !res || ori_h <= 0 || ori_w <= 0) return 1;
    if (!c->net->upload_image(image_chw)) return 2;
    const auto t0 = std::chrono::steady_clock::now();
    if (c->net->replay() != 0) {
        fprintf(stderr, "ppdl: graph compute failed\n");
        return 2;
    }
    const auto t1 = std::chrono::steady_clock::now();
    c->computed = true;
    c->fetched = false;
    if (!c->net->download(c->host.logits, c->host.boxes, c->host.order, c->host.mbits)) return 2;
    ppdl::assemble_result(c->host, ori_h, ori_w, c->dets, c->masks, c->picks);
    c->fetched = true;
    res->dets = c->dets.data();
    res->num_dets = ppdl::NQ;
    res->masks = c->masks.data();
    res->infer_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    return 0;
}

extern "C" PPDL_API int ppdl_dump(ppdl_ctx *c, const char *dir) {
    if (!c || !dir) return 1;
    if (c->net->dumps_.empty()) {
        fprintf(stderr, "ppdl: dumps not enabled\n");
        return 1;
    }
    if (!c->computed) {
        fprintf(stderr, "ppdl: no inference to dump\n");
        return 1;
    }
    mkdir(dir, 0755);
    FILE *mf = fopen((std::string(dir) + "/shapes.txt").c_str(), "w");
    if (!mf) return 1;
    for (const auto &d : c->net->dumps_) {
        int64_t n = 1;
        for (int64_t e : d.ne) n *= e;
        std::vector<uint8_t> buf((size_t)n * 4);
        if (hipMemcpy(buf.data(), d.d, buf.size(), hipMemcpyDeviceToHost) != hipSuccess) {
            fclose(mf);
            return 1;
        }
        ppdl::write_file(std::string(dir) + "/" + d.name + ".bin", buf.data(), buf.size());
        std::vector<int64_t> ne = d.ne;
        while (ne.size() < 4) ne.push_back(1);
        fprintf(mf, "%s %s %lld %lld %lld %lld\n", d.name.c_str(), d.i32 ? "i32" : "f32", (long long)ne[0],
                (long long)ne[1], (long long)ne[2], (long long)ne[3]);
    }
    fclose(mf);
    return 0;
}

extern "C" PPDL_API int ppdl_dump_raw(ppdl_ctx *c, const char *pfx) {
    if (!c || !pfx) return 1;
    if (!c->fetched) {
        fprintf(stderr, "ppdl: no inference to dump\n");
        return 1;
    }
    using ppdl::NQ;
    using ppdl::NC;
    const std::string p(pfx);
    bool good = ppdl::write_file(p + "logits.bin", c->host.logits, (size_t)NQ * NC * 4);
    good = ppdl::write_file(p + "boxes.bin", c->host.boxes, (size_t)NQ * 4 * 4) && good;
    good = ppdl::write_file(p + "order.bin", c->host.order, (size_t)NQ * NQ * 4) && good;
    good = ppdl::write_file(p + "sel.bin", c->picks.data(), c->picks.size() * 4) && good;
    return good ? 0 : 1;
}

extern "C" PPDL_API void ppdl_free(ppdl_ctx *c) { delete c; }

extern "C" PPDL_API int64_t ppdl_get_raw(ppdl_ctx *c, int which, void *dst, int64_t n) {
    using namespace ppdl;
    if (!c || !dst || !c->computed) return -1;
    const void *src = nullptr;
    int64_t cnt = 0;
    switch (which) {
        case 0: src = c->net->logits_; cnt = (int64_t)NQ * NC; break;
        case 1: src = c->net->boxes_; cnt = (int64_t)NQ * 4; break;
        case 2: src = c->net->order_; cnt = (int64_t)NQ * NQ; break;
        case 3:
            // the final mask logits: the graph keeps only their signs, so the
            // same GEMM runs once more without the bits, on the graph's inputs
            if (!c->net->mask_logits()) return -1;
            src = c->net->masks_;
            cnt = (int64_t)NQ * NPIX;
            break;
        case 4: src = c->net->topk_; cnt = NQ; break;
        case 5: src = c->net->refu_; cnt = (int64_t)NQ * 4; break;
        default: return -1;
    }
    if (n < cnt) return -1;
    return hipMemcpy(dst, src, (size_t)cnt * 4, hipMemcpyDeviceToHost) == hipSuccess ? cnt : -1;
}

extern "C" PPDL_API double ppdl_time_graph(ppdl_ctx *c, int iters) {
    if (!c) return -1.0;
    return c->net->time_graph(iters);
}

extern "C" PPDL_API int ppdl_graph_nodes(ppdl_ctx *c) { return c ? c->net->nodes() : 0; }

extern "C" PPDL_API int ppdl_profile_nodes(ppdl_ctx *c, int iters, ppdl_node_stat *out, int cap) {
    if (!c || !out || cap < 1) return -1;
    return c->net->profile_nodes(iters, out, cap);
}
