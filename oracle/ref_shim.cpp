// oracle/ref_shim.cpp - exports the reference's own header-only codecs and IQ2_S codebook with C linkage,
// so tests can pin the oracle's restatements against the reference itself.  Compiled by oracle/Makefile
// against the headers where they lie under /root/reference; nothing of the reference is copied here.
//   include/strata/kernels/f16_bits.hpp:37-101   f16_from_f32 / f32_from_f16
//   include/strata/kernels/bf16_bits.hpp:37-59   bf16_from_f32 / f32_from_bf16
//   include/strata/artifact/dequant.hpp:69-78    dequantize_q2_0
//   include/strata/artifact/dequant.hpp:81-280   the other native types (Q8_0, Q4_0, Q5_0, IQ4_NL, Q6_K, Q4_K,
//                                                Q5_K, Q3_K, IQ4_XS)
//   metal/include/strata/metal/iq_grids.hpp:5    iq2s_grid
//   include/strata/artifact/gguf_reader.hpp       GgufModel (GgufFile, split shards, tensor_payload_bytes)
#include "strata/artifact/dequant.hpp"
#include "strata/artifact/gguf_reader.hpp"
#include "strata/kernels/bf16_bits.hpp"
#include "strata/kernels/f16_bits.hpp"
#include "strata/metal/iq_grids.hpp"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

extern "C" {
uint16_t ref_f16_from_f32(float f) { return strata::kernels::f16_from_f32(f); }
float ref_f32_from_f16(uint16_t h) { return strata::kernels::f32_from_f16(h); }
uint16_t ref_bf16_from_f32(float f) { return strata::kernels::bf16_from_f32(f); }
float ref_f32_from_bf16(uint16_t h) { return strata::kernels::f32_from_bf16(h); }
void ref_f16_from_f32_n(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::f16_from_f32(x[i]);
}
void ref_bf16_from_f32_n(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::bf16_from_f32(x[i]);
}
void ref_f32_from_f16_all(float* out65536) {
    for (uint32_t h = 0; h < 65536u; ++h) out65536[h] = strata::kernels::f32_from_f16((uint16_t) h);
}
void ref_dequantize_q2_0(const uint8_t* blocks, int64_t n_blocks, float* out) {
    for (int64_t b = 0; b < n_blocks; ++b) strata::dequantize_q2_0(blocks + b * 18, out + b * 64);
}
// n_values of ggml `type` from its blocks; returns -1 for a type the reference does not dequantise here
int ref_dequantize(int type, const uint8_t* blocks, int64_t n_values, float* out) {
    int qk = 0, bytes = 0;
    void (*fn)(const uint8_t*, float*) = nullptr;
    switch (type) {
        case 8: qk = 32; bytes = 34; fn = strata::dequantize_q8_0; break;
        case 2: qk = 32; bytes = 18; fn = strata::dequantize_q4_0; break;
        case 6: qk = 32; bytes = 22; fn = strata::dequantize_q5_0; break;
        case 20: qk = 32; bytes = 18; fn = strata::dequantize_iq4_nl; break;
        case 23: qk = 256; bytes = 136; fn = strata::dequantize_iq4_xs; break;
        case 11: qk = 256; bytes = 110; fn = strata::dequantize_q3_K; break;
        case 12: qk = 256; bytes = 144; fn = strata::dequantize_q4_K; break;
        case 13: qk = 256; bytes = 176; fn = strata::dequantize_q5_K; break;
        case 14: qk = 256; bytes = 210; fn = strata::dequantize_q6_K; break;
        default: return -1;
    }
    if (n_values % qk) return -1;
    for (int64_t b = 0; b < n_values / qk; ++b) fn(blocks + b * bytes, out + b * qk);
    return 0;
}
void ref_iq2s_grid(uint64_t* out1024) { std::memcpy(out1024, strata::metal::iq2s_grid, sizeof(strata::metal::iq2s_grid)); }
// The reference reader's view of a model (any shard's path): per shard "shard <i> <data_start> <n_tensors>", then per
// tensor "<name> <type> <n_dims> <ne...> <offset> <payload bytes> <in bounds>"; -1 with "ERR <why>" when it refuses.
int ref_gguf_list(const char* path, char* out, size_t cap) {
    try {
        strata::GgufModel m = strata::GgufModel::open(path);
        std::string s;
        for (size_t i = 0; i < m.size(); ++i) {
            const strata::GgufFile& f = m.shard(i);
            s += "shard " + std::to_string(i) + " " + std::to_string(f.data_start()) + " " +
                 std::to_string(f.tensors().size()) + "\n";
            for (const auto& t : f.tensors()) {
                s += t.name + " " + std::to_string(t.type) + " " + std::to_string(t.shape.size());
                for (uint64_t d : t.shape) s += " " + std::to_string(d);
                s += " " + std::to_string(t.offset) + " " + std::to_string(strata::tensor_payload_bytes(t)) + " " +
                     (m.in_bounds(t, i) ? "1" : "0") + "\n";
            }
        }
        if (s.size() + 1 > cap) return -2;
        std::memcpy(out, s.c_str(), s.size() + 1);
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(out, cap, "ERR %s", e.what());
        return -1;
    }
}
}
