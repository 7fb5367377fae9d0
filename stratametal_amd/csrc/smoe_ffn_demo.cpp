// stratametal_amd/csrc/smoe_ffn_demo.cpp - the C++ operator (include/smoe_ffn.hpp) end to end: a seeded
// synthetic layer generated on the device (the same streams as stratametal_amd.synth_layer: 1 gate, 2 up,
// 3 down, 4 router, 5/6/7 shared gate/up/down, 8 shared gate_inp; x from stream 100), one traced
// FfnExec::run, and the trace written to a file for the host check; then the whole layer call (run_layer) on 4
// residual streams with hc_lr 320 (hyper-connection tensors from streams 30 norm = 1 + N(0, 0.1^2), 31 down and
// 32 up N(0, 0.2^2), 33 inject N(0, 0.05^2); the streams from stream 101).
//
//   smoe_ffn_demo OUT n_tokens seed n_embd n_ff n_ff_shared n_expert top_k
//
// OUT receives, little-endian: int32 T, H, E, K; f32 combined [T][H]; int32 ids [T][K]; f32 route_w [T][K];
// int32 counts [E]; f32 stage_ms [5]; f32 layer output [T][4][H].
//
//   smoe_ffn_demo --gguf OUT MODEL layer n_tokens seed n_embd n_ff n_expert hc hc_lr with_shared
//
// The same from a GGUF model: FfnExec::load(model, layer, geometry, with_shared) (top_k from the model), x from
// stream 100; OUT as above, the layer output [T][hc][H] (residual streams from stream 101) when hc > 0.
#include "smoe_ffn.hpp"

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {
void* dev_alloc(size_t bytes) {
    void* p = nullptr;
    smoe::check_hip(hipMalloc(&p, bytes), "hipMalloc");
    return p;
}
size_t block_bytes(int32_t type, int64_t n) { return type == SMOE_Q2_0 ? n / 64 * 18 : n / 256 * 82; }

void write_out(const char* path, int32_t T, const smoe_geom& g, const smoe::FfnTrace& tr, const std::vector<float>& layer) {
    FILE* f = std::fopen(path, "wb");
    if (!f) throw std::runtime_error(std::string("cannot open ") + path);
    const int32_t hdr[4] = {T, g.n_embd, g.n_expert, g.top_k};
    std::fwrite(hdr, 4, 4, f);
    std::fwrite(tr.combined.data(), 4, tr.combined.size(), f);
    std::fwrite(tr.ids.data(), 4, tr.ids.size(), f);
    std::fwrite(tr.route_w.data(), 4, tr.route_w.size(), f);
    std::fwrite(tr.counts.data(), 4, tr.counts.size(), f);
    std::fwrite(tr.stage_ms.data(), 4, tr.stage_ms.size(), f);
    std::fwrite(layer.data(), 4, layer.size(), f);
    std::fclose(f);
}

int from_gguf(int argc, char** argv) {
    if (argc != 13) {
        std::fprintf(stderr, "usage: %s --gguf OUT MODEL layer n_tokens seed n_embd n_ff n_expert hc hc_lr with_shared\n",
                     argv[0]);
        return 2;
    }
    const char* out_path = argv[2];
    const int32_t layer = std::atoi(argv[4]), T = std::atoi(argv[5]);
    const uint64_t seed = std::strtoull(argv[6], nullptr, 10);
    smoe::ModelGeometry mg;
    mg.n_embd = std::atoll(argv[7]);
    mg.n_ff = std::atoll(argv[8]);
    mg.n_expert = std::atoll(argv[9]);
    mg.hc = std::atoll(argv[10]);
    mg.hc_lr = std::atoll(argv[11]);
    const bool with_shared = std::atoi(argv[12]) != 0;
    smoe_model* m = nullptr;
    smoe::check(smoe_model_open(argv[3], &m), "smoe_model_open");
    smoe::FfnExec ffn;
    try {
        ffn = smoe::FfnExec::load(m, layer, mg, with_shared, T, /*with_trace*/ true);
    } catch (...) {
        smoe_model_close(m);
        throw;
    }
    smoe_model_close(m);  // the operator's device copies outlive the mapping
    const smoe_geom& g = ffn.geom();
    float* x = static_cast<float*>(dev_alloc((size_t)T * g.n_embd * 4));
    float* y = static_cast<float*>(dev_alloc((size_t)T * g.n_embd * 4));
    smoe::check(smoe_synth_normal(seed, 100, (int64_t)T * g.n_embd, 1.0f, x, nullptr), "synth x");
    smoe::FfnTrace tr;
    ffn.run(x, y, T, /*add_shared*/ with_shared, &tr);
    std::vector<float> layer_h;
    if (mg.hc > 0) {
        const int64_t hd = mg.hc * g.n_embd;
        float* R = static_cast<float*>(dev_alloc((size_t)T * hd * 4));
        float* out = static_cast<float*>(dev_alloc((size_t)T * hd * 4));
        smoe::check(smoe_synth_normal(seed, 101, (int64_t)T * hd, 1.0f, R, nullptr), "synth residual");
        ffn.run_layer(R, out, T, /*add_shared*/ with_shared);
        layer_h.resize((size_t)T * hd);
        smoe::check_hip(hipMemcpy(layer_h.data(), out, layer_h.size() * 4, hipMemcpyDeviceToHost), "layer output copy");
    }
    write_out(out_path, T, g, tr, layer_h);
    std::printf("FfnExec from layer %d of %s: %d tokens, top_k %d, %llu device bytes owned\n", layer, argv[3], T,
                g.top_k, (unsigned long long)ffn.gpu_bytes());
    return 0;
}
}  // namespace

int main(int argc, char** argv) {
    if (argc > 1 && std::string(argv[1]) == "--gguf") {
        try {
            return from_gguf(argc, argv);
        } catch (const std::exception& e) {
            std::fprintf(stderr, "smoe_ffn_demo: %s\n", e.what());
            return 1;
        }
    }
    if (argc != 9) {
        std::fprintf(stderr, "usage: %s OUT n_tokens seed n_embd n_ff n_ff_shared n_expert top_k\n", argv[0]);
        return 2;
    }
    try {
        const int32_t T = std::atoi(argv[2]);
        const uint64_t seed = std::strtoull(argv[3], nullptr, 10);
        smoe_geom g{};
        g.n_embd = std::atoi(argv[4]);
        g.n_ff = std::atoi(argv[5]);
        g.n_ff_shared = std::atoi(argv[6]);
        g.n_expert = std::atoi(argv[7]);
        g.top_k = std::atoi(argv[8]);
        g.w_type = SMOE_Q2_0;
        g.sh_type = SMOE_Q2_0;
        g.router_dtype = 0;
        const int64_t H = g.n_embd, F = g.n_ff, Fs = g.n_ff_shared, E = g.n_expert;
        const float sigma = 0.02f;
        auto blocks = [&](uint64_t stream_id, int64_t n) {
            void* p = dev_alloc(block_bytes(SMOE_Q2_0, n));
            smoe::check(smoe_synth_blocks(SMOE_Q2_0, seed, stream_id, n, sigma, p, nullptr), "synth blocks");
            return p;
        };
        auto bf16 = [&](uint64_t stream_id, int64_t n) {
            void* p = dev_alloc((size_t)n * 2);
            smoe::check(smoe_synth_bf16(seed, stream_id, n, sigma, static_cast<uint16_t*>(p), nullptr), "synth bf16");
            return static_cast<const uint16_t*>(p);
        };
        smoe_weights w{};
        w.gate_exps = blocks(1, E * F * H);
        w.up_exps = blocks(2, E * F * H);
        w.down_exps = blocks(3, E * H * F);
        w.router = bf16(4, E * H);
        w.gate_sh = blocks(5, Fs * H);
        w.up_sh = blocks(6, Fs * H);
        w.down_sh = blocks(7, H * Fs);
        w.gate_inp_sh = bf16(8, H);
        float* x = static_cast<float*>(dev_alloc((size_t)T * H * 4));
        float* y = static_cast<float*>(dev_alloc((size_t)T * H * 4));
        smoe::check(smoe_synth_normal(seed, 100, (int64_t)T * H, 1.0f, x, nullptr), "synth x");

        const int32_t hc_n = 4, hc_lr = 320;
        const int64_t hd = (int64_t)hc_n * H;
        std::vector<float> norm_h((size_t)hd);
        float* norm = static_cast<float*>(dev_alloc((size_t)hd * 4));
        smoe::check(smoe_synth_normal(seed, 30, hd, 0.1f, norm, nullptr), "synth hc norm");
        smoe::check_hip(hipMemcpy(norm_h.data(), norm, (size_t)hd * 4, hipMemcpyDeviceToHost), "norm copy");
        for (float& v : norm_h) v = 1.0f + v;  // the stored (1 + w)
        smoe::check_hip(hipMemcpy(norm, norm_h.data(), (size_t)hd * 4, hipMemcpyHostToDevice), "norm copy");
        auto bf16_s = [&](uint64_t stream_id, int64_t n, float s) {
            void* p = dev_alloc((size_t)n * 2);
            smoe::check(smoe_synth_bf16(seed, stream_id, n, s, static_cast<uint16_t*>(p), nullptr), "synth bf16");
            return static_cast<const uint16_t*>(p);
        };
        smoe_hc hc{hc_n, hc_lr, 1e-6f, norm, bf16_s(31, hc_lr * hd, 0.2f), bf16_s(32, hd * hc_lr, 0.2f),
                   bf16_s(33, hc_n * hd, 0.05f)};
        float* R = static_cast<float*>(dev_alloc((size_t)T * hd * 4));
        float* out = static_cast<float*>(dev_alloc((size_t)T * hd * 4));
        smoe::check(smoe_synth_normal(seed, 101, (int64_t)T * hd, 1.0f, R, nullptr), "synth residual");

        smoe::FfnExec ffn = smoe::FfnExec::load(g, w, T, /*with_trace*/ true, &hc);
        smoe::FfnTrace tr;
        ffn.run(x, y, T, /*add_shared*/ true, &tr);
        ffn.run_layer(R, out, T, /*add_shared*/ true);
        std::vector<float> out_h((size_t)T * hd);
        smoe::check_hip(hipMemcpy(out_h.data(), out, out_h.size() * 4, hipMemcpyDeviceToHost), "layer output copy");

        write_out(argv[1], T, g, tr, out_h);
        std::printf("FfnExec: %d tokens, %llu device bytes owned, stages (ms):", T, (unsigned long long)ffn.gpu_bytes());
        for (float m : tr.stage_ms) std::printf(" %.4f", m);
        std::printf("\n");
    } catch (const std::exception& e) {
        std::fprintf(stderr, "smoe_ffn_demo: %s\n", e.what());
        return 1;
    }
    return 0;
}
