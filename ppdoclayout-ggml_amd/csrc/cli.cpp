// Command-line front end over the C API (include/ppdoclayout.h), with the
// reference CLI's flags and output files (src/main.cpp:37-133 of the
// reference):
//
//   ppdoclayout -m model.gguf -i input.bin [--ori-h H] [--ori-w W] [-o outdir]
//               [--backend hip|cuda] [--bench N] [--dump-dir d] [--dump-raw pfx]
//   ppdoclayout -m model.gguf --batch manifest      (lines "in.bin|outdir|H|W")
//
// input.bin holds the float32 CHW 3x800x800 page (RGB, /255).  Writes
// outdir/out0.bin (300x7 f32 detections), out1.bin (i32 detection count),
// out2.bin (300x200x200 i32 masks); batch mode writes out0/out2 per line.
// `--backend cpu` is refused: this build has only the GPU backend.
#include <sys/stat.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ppdoclayout.h"

namespace {

constexpr size_t kImgFloats = (size_t)3 * PPDL_IMG_SIZE * PPDL_IMG_SIZE;

bool load_bytes(const char *path, void *dst, size_t n) {
    FILE *f = fopen(path, "rb");
    if (!f) return false;
    const size_t got = fread(dst, 1, n, f);
    fclose(f);
    return got == n;
}

bool save_bytes(const std::string &path, const void *src, size_t n) {
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) return false;
    const size_t put = fwrite(src, 1, n, f);
    return fclose(f) == 0 && put == n;
}

bool save_result(const std::string &dir, const ppdl_result &r, bool with_count) {
    mkdir(dir.c_str(), 0755);
    bool good = save_bytes(dir + "/out0.bin", r.dets, (size_t)r.num_dets * PPDL_DET_FIELDS * sizeof(float));
    if (with_count) good = good && save_bytes(dir + "/out1.bin", &r.num_dets, sizeof(int32_t));
    good = good && save_bytes(dir + "/out2.bin", r.masks,
                              (size_t)r.num_dets * PPDL_MASK_HW * PPDL_MASK_HW * sizeof(int32_t));
    return good;
}

int usage() {
    fprintf(stderr,
            "usage: ppdoclayout -m model.gguf -i input.bin [--ori-h H] [--ori-w W] [-o outdir] "
            "[--backend hip|cuda] [--bench N] [--dump-dir d] [--dump-raw pfx] | --batch manifest\n");
    return 1;
}

// manifest lines "in.bin|outdir|ori_h|ori_w"; the model is loaded once
int run_batch(ppdl_ctx *ctx, const char *manifest) {
    FILE *mf = fopen(manifest, "r");
    if (!mf) {
        fprintf(stderr, "cannot open %s\n", manifest);
        return 1;
    }
    std::vector<float> img(kImgFloats);
    char line[2048];
    int done = 0, failed = 0;
    while (fgets(line, sizeof(line), mf)) {
        char in[1000], od[1000];
        int h = 0, w = 0;
        if (sscanf(line, "%999[^|]|%999[^|]|%d|%d", in, od, &h, &w) != 4) continue;
        ppdl_result r;
        if (!load_bytes(in, img.data(), img.size() * sizeof(float))) {
            fprintf(stderr, "read fail %s\n", in);
            failed++;
        } else if (ppdl_infer(ctx, img.data(), h, w, &r) != 0) {
            fprintf(stderr, "infer fail %s\n", in);
            failed++;
        } else if (!save_result(od, r, false)) {
            fprintf(stderr, "write fail %s\n", od);
            failed++;
        } else {
            done++;
        }
    }
    fclose(mf);
    fprintf(stderr, "batch: %d done, %d failed\n", done, failed);
    return failed ? 1 : 0;
}

}  // namespace

int main(int argc, char **argv) {
    const char *model = "model-f32.gguf", *input = nullptr, *out_dir = ".", *dump_dir = nullptr;
    const char *dump_raw = nullptr, *manifest = nullptr;
    std::string backend = "hip";
    int ori_h = PPDL_IMG_SIZE, ori_w = PPDL_IMG_SIZE, bench = 0;
    for (int i = 1; i < argc; i++) {
        const std::string a = argv[i];
        if (i + 1 >= argc) {
            fprintf(stderr, "missing value for %s\n", a.c_str());
            return 1;
        }
        const char *v = argv[++i];
        if (a == "-m") model = v;
        else if (a == "-i") input = v;
        else if (a == "-o") out_dir = v;
        else if (a == "--ori-h") ori_h = atoi(v);
        else if (a == "--ori-w") ori_w = atoi(v);
        else if (a == "--backend") backend = v;
        else if (a == "--bench") bench = atoi(v);
        else if (a == "--dump-dir") dump_dir = v;
        else if (a == "--dump-raw") dump_raw = v;
        else if (a == "--batch") manifest = v;
        else {
            fprintf(stderr, "unknown arg: %s\n", a.c_str());
            return 1;
        }
    }
    if (!input && !manifest) return usage();
    int be;
    if (backend == "hip") be = PPDL_BACKEND_HIP;
    else if (backend == "cuda") be = PPDL_BACKEND_CUDA;
    else {
        fprintf(stderr, "backend '%s' is not available in this build (hip only)\n", backend.c_str());
        return 1;
    }

    ppdl_ctx *ctx = ppdl_init_ex(model, be, dump_dir != nullptr);
    if (!ctx) return 1;
    int rc = 0;
    if (manifest) {
        rc = run_batch(ctx, manifest);
    } else {
        std::vector<float> img(kImgFloats);
        ppdl_result r;
        if (!load_bytes(input, img.data(), img.size() * sizeof(float))) {
            fprintf(stderr, "failed to read %s\n", input);
            rc = 1;
        } else if (ppdl_infer(ctx, img.data(), ori_h, ori_w, &r) != 0) {
            rc = 1;
        } else {
            fprintf(stderr, "inference: %.1f ms\n", r.infer_ms);
            if (bench > 0) {
                double sum = 0.0, sq = 0.0;
                for (int i = 0; i < bench && rc == 0; i++) {
                    if (ppdl_infer(ctx, img.data(), ori_h, ori_w, &r) != 0) rc = 1;
                    sum += r.infer_ms;
                    sq += r.infer_ms * r.infer_ms;
                }
                const double mean = sum / bench;
                printf("bench_ms mean=%.2f std=%.2f n=%d\n", mean, std::sqrt(std::fmax(sq / bench - mean * mean, 0.0)),
                       bench);
            }
            if (rc == 0 && dump_dir && ppdl_dump(ctx, dump_dir) != 0) rc = 1;
            if (rc == 0 && dump_raw && ppdl_dump_raw(ctx, dump_raw) != 0) rc = 1;
            if (rc == 0) {
                if (!save_result(out_dir, r, true)) rc = 1;
                else fprintf(stderr, "wrote %s/out0.bin out1.bin out2.bin\n", out_dir);
            }
        }
    }
    ppdl_free(ctx);
    return rc;
}
