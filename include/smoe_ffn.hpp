// include/smoe_ffn.hpp - the C++ FfnExec-shaped operator over the C ABI in smoe.h (header-only).
//
// Mirrors the reference's per-layer feed-forward operator, FfnExec::load / FfnExec::run
// (metal/include/strata/metal/layer_exec.hpp:113-140): run() is its MoE interior (metal/src/layer_exec.cpp:470-530,
// `mixed` to `combined`), run_layer() the whole call with the hyper-connection ends around it; load() takes the
// layer's device tensors and geometry, or the layer of an open GGUF model and the model geometry, once and owns
// every buffer the call needs, sized for a maximum token count, so that run() allocates nothing; status codes become
// exceptions (the reference throws MetalError, metal/include/strata/metal/device.hpp:28-31); a traced run
// copies the stage outputs to host vectors, as FfnTrace does (layer_exec.hpp:100-109).  Uses only smoe.h and
// the HIP runtime.
#pragma once

#include "smoe.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace smoe {

// A refused or failed call: the smoe_status and the library's reason.
struct Error : std::runtime_error {
    smoe_status status;
    Error(smoe_status s, const std::string& what) : std::runtime_error(what), status(s) {}
};

inline void check(smoe_status s, const char* where) {
    if (s != SMOE_OK) throw Error(s, std::string(where) + ": " + smoe_status_str(s) + ": " + smoe_last_error());
}
inline void check_hip(hipError_t e, const char* where) {
    if (e != hipSuccess) throw Error(SMOE_EDEVICE, std::string(where) + ": " + hipGetErrorString(e));
}

// What one MoE pass produced, on the host (the MoE fields of the reference's FfnTrace, same names where they
// correspond: route = router logits, route_w = routing weights, sgate = the shared expert's gate dot).
struct FfnTrace {
    std::vector<float> mixed, combined;  // [T][n_embd] input and output
    std::vector<float> route;            // [T][n_expert]
    std::vector<int32_t> ids;            // [T][k], selection order
    std::vector<float> route_w;          // [T][k]
    std::vector<float> sgate;            // [T] (before the sigmoid)
    std::vector<int32_t> counts, offsets, perm, slot;  // the dispatch: [E], [E+1], [T*k], [T*k]
    std::vector<float> stage_ms;         // router, route, gate/up, down, combine
};

// The MoE and hyper-connection fields of the reference's model geometry (strata::core::ModelGeometry,
// include/strata/core/layout.hpp:27-55) that a layer's tensors must match; hc 0: no check of the hyper-connection
// shapes.
struct ModelGeometry {
    int64_t n_embd = 0, n_ff = 0, n_expert = 0;
    int64_t hc = 0, hc_lr = 0;
};

class FfnExec {
   public:
    // The reference's FfnExec::load(model, layer, geometry, with_shared) (metal/src/layer_exec.cpp:369-452): layer
    // `layer`'s MoE tensors from an open model (smoe_model_open: blk.<layer>.ffn_{gate,up,down}_exps,
    // ffn_gate_inp, with_shared the shared expert's planes and gate, and the hyper-connection tensors when the
    // file has them), checked against `geom` (a routed plane of another shape is refused, as the reference's
    // expert_spans refuses it), copied into device memory this operator owns, and the operator loaded on them for
    // up to `max_tokens` tokens per run.  top_k 0: the model's <arch>.expert_used_count.  The copies are
    // complete when load returns (the mapping may be closed after).
    static FfnExec load(const smoe_model* model, int32_t layer, const ModelGeometry& geom, bool with_shared,
                        int32_t max_tokens, bool with_trace = false, int32_t top_k = 0, hipStream_t stream = nullptr) {
        smoe_layer_plan plan{};
        check(smoe_layer_plan_for(model, layer, top_k, with_shared ? 1 : 0, &plan), "FfnExec::load plan");
        const smoe_geom& g = plan.geom;
        auto mismatch = [&](const char* what, int64_t have, int64_t want) {
            if (have != want)
                throw Error(SMOE_EINVAL, "FfnExec::load: layer " + std::to_string(layer) + " has " + what + " " +
                                             std::to_string(have) + ", the geometry says " + std::to_string(want));
        };
        mismatch("n_embd", g.n_embd, geom.n_embd);
        mismatch("n_ff", g.n_ff, geom.n_ff);
        mismatch("n_expert", g.n_expert, geom.n_expert);
        if (geom.hc > 0) {
            mismatch("hc", plan.hc.hc, geom.hc);
            mismatch("hc_lr", plan.hc.hc_lr, geom.hc_lr);
        }
        void* buf = nullptr;
        check_hip(hipMalloc(&buf, plan.device_bytes), "FfnExec::load weights");
        try {
            smoe_weights w{};
            smoe_hc hc{};
            const bool has_hc = plan.hc.hc > 0;
            check(smoe_layer_upload(model, &plan, buf, plan.device_bytes, &w, has_hc ? &hc : nullptr, stream),
                  "FfnExec::load upload");
            FfnExec f = load(g, w, max_tokens, with_trace, has_hc ? &hc : nullptr);
            f.wbuf_ = buf;
            f.wbuf_bytes_ = plan.device_bytes;
            return f;
        } catch (...) {
            (void)hipFree(buf);
            throw;
        }
    }

    // The layer's tensors (device pointers into the loaded model, e.g. a GGUF mapping) and geometry; buffers
    // for up to `max_tokens` tokens per run, and for tracing when `with_trace`.
    // With `hc` (the layer's hyper-connection tensors) the operator also runs the whole layer call, run_layer.
    static FfnExec load(const smoe_geom& geom, const smoe_weights& weights, int32_t max_tokens, bool with_trace = false,
                        const smoe_hc* hc = nullptr) {
        FfnExec f;
        f.g_ = geom;
        f.w_ = weights;
        f.max_tokens_ = max_tokens;
        if (hc) {
            f.hc_ = *hc;
            f.has_hc_ = true;
        }
        // the layer call's workspace begins with the block's own, so one buffer serves run and run_layer
        f.ws_bytes_ = hc ? smoe_ffn_workspace_bytes(&f.g_, hc, max_tokens) : smoe_workspace_bytes(&f.g_, max_tokens);
        if (f.ws_bytes_ == 0) throw Error(SMOE_EINVAL, std::string("FfnExec::load: ") + smoe_last_error());
        check_hip(hipMalloc(&f.ws_, f.ws_bytes_), "FfnExec::load workspace");
        if (with_trace) {
            const size_t T = (size_t)max_tokens, E = (size_t)geom.n_expert, K = (size_t)geom.top_k;
            f.tr_bytes_ = 4 * (T * E + 2 * T * K + E + (E + 1) + 2 * T * K + T);
            check_hip(hipMalloc(&f.tr_, f.tr_bytes_), "FfnExec::load trace");
            for (hipEvent_t& e : f.ev_) check_hip(hipEventCreate(&e), "FfnExec::load events");
        }
        return f;
    }

    FfnExec() = default;
    FfnExec(const FfnExec&) = delete;
    FfnExec& operator=(const FfnExec&) = delete;
    FfnExec(FfnExec&& o) noexcept { *this = std::move(o); }
    FfnExec& operator=(FfnExec&& o) noexcept {
        if (this != &o) {
            release();
            g_ = o.g_;
            w_ = o.w_;
            hc_ = o.hc_;
            has_hc_ = o.has_hc_;
            max_tokens_ = o.max_tokens_;
            ws_ = std::exchange(o.ws_, nullptr);
            ws_bytes_ = std::exchange(o.ws_bytes_, 0);
            tr_ = std::exchange(o.tr_, nullptr);
            tr_bytes_ = std::exchange(o.tr_bytes_, 0);
            wbuf_ = std::exchange(o.wbuf_, nullptr);
            wbuf_bytes_ = std::exchange(o.wbuf_bytes_, 0);
            for (int i = 0; i < SMOE_STAGE_EVENTS; ++i) ev_[i] = std::exchange(o.ev_[i], nullptr);
        }
        return *this;
    }
    ~FfnExec() { release(); }

    // combined[T][n_embd] = MoE(mixed[T][n_embd]) (device pointers), the shared expert added when `add_shared`.
    // Enqueued on `stream`; a traced run (`trace` non-null, load(with_trace)) waits for it and fills `trace`.
    void run(const float* mixed, float* combined, int32_t n_tokens, bool add_shared, FfnTrace* trace = nullptr,
             hipStream_t stream = nullptr) {
        if (n_tokens > max_tokens_)
            throw Error(SMOE_ESIZE, "FfnExec::run: " + std::to_string(n_tokens) + " tokens, loaded for " +
                                        std::to_string(max_tokens_));
        if (trace && !tr_) throw Error(SMOE_EINVAL, "FfnExec::run: traced run of an operator loaded without tracing");
        smoe_trace t{};
        void* events[SMOE_STAGE_EVENTS];
        if (trace) {
            t = trace_ptrs();
            for (int i = 0; i < SMOE_STAGE_EVENTS; ++i) events[i] = ev_[i];
            t.stage_events = events;
        }
        check(smoe_forward(&g_, &w_, mixed, n_tokens, combined, add_shared ? 1 : 0, ws_, ws_bytes_,
                           trace ? &t : nullptr, stream),
              "FfnExec::run");
        if (!trace) return;
        check_hip(hipStreamSynchronize(stream), "FfnExec::run sync");
        const size_t T = (size_t)n_tokens, H = (size_t)g_.n_embd, E = (size_t)g_.n_expert, K = (size_t)g_.top_k;
        auto get = [](auto& v, const void* src, size_t n) {
            v.resize(n);
            check_hip(hipMemcpy(v.data(), src, n * sizeof(v[0]), hipMemcpyDeviceToHost), "FfnExec trace copy");
        };
        get(trace->mixed, mixed, T * H);
        get(trace->combined, combined, T * H);
        get(trace->route, t.logits, T * E);
        get(trace->ids, t.ids, T * K);
        get(trace->route_w, t.weights, T * K);
        get(trace->counts, t.counts, E);
        get(trace->offsets, t.offsets, E + 1);
        get(trace->perm, t.perm, T * K);
        get(trace->slot, t.slot, T * K);
        if (g_.sh_type >= 0) get(trace->sgate, t.sgate, T);
        else trace->sgate.clear();
        trace->stage_ms.assign(SMOE_STAGE_EVENTS - 1, 0.0f);
        for (int i = 0; i + 1 < SMOE_STAGE_EVENTS; ++i)
            check_hip(hipEventElapsedTime(&trace->stage_ms[i], ev_[i], ev_[i + 1]), "FfnExec stage time");
    }

    // The whole layer call of the reference's FfnExec::run(residual, out, add_shared) (metal/src/layer_exec.cpp:
    // 462-531): gr_read of the residual streams [T][hc][n_embd], the MoE block, gr_write of its output onto every
    // stream into out (which may be residual).  Needs load(..., hc).
    void run_layer(const float* residual, float* out, int32_t n_tokens, bool add_shared, hipStream_t stream = nullptr) {
        if (!has_hc_) throw Error(SMOE_EINVAL, "FfnExec::run_layer: operator loaded without hyper-connection tensors");
        if (n_tokens > max_tokens_)
            throw Error(SMOE_ESIZE, "FfnExec::run_layer: " + std::to_string(n_tokens) + " tokens, loaded for " +
                                        std::to_string(max_tokens_));
        check(smoe_ffn_run(&g_, &w_, &hc_, residual, n_tokens, out, add_shared ? 1 : 0, ws_, ws_bytes_, nullptr,
                           stream),
              "FfnExec::run_layer");
    }

    // Device bytes this operator owns (workspace and trace buffers, and the layer's tensors when it loaded them
    // from a model; otherwise the weights are the caller's).
    uint64_t gpu_bytes() const { return ws_bytes_ + tr_bytes_ + wbuf_bytes_; }
    const smoe_geom& geom() const { return g_; }

   private:
    smoe_trace trace_ptrs() const {
        const size_t T = (size_t)max_tokens_, E = (size_t)g_.n_expert, K = (size_t)g_.top_k;
        char* p = static_cast<char*>(tr_);
        smoe_trace t{};
        t.logits = reinterpret_cast<float*>(p);
        p += 4 * T * E;
        t.ids = reinterpret_cast<int32_t*>(p);
        p += 4 * T * K;
        t.weights = reinterpret_cast<float*>(p);
        p += 4 * T * K;
        t.counts = reinterpret_cast<int32_t*>(p);
        p += 4 * E;
        t.offsets = reinterpret_cast<int32_t*>(p);
        p += 4 * (E + 1);
        t.perm = reinterpret_cast<int32_t*>(p);
        p += 4 * T * K;
        t.slot = reinterpret_cast<int32_t*>(p);
        p += 4 * T * K;
        t.sgate = g_.sh_type >= 0 ? reinterpret_cast<float*>(p) : nullptr;
        return t;
    }
    void release() noexcept {
        if (ws_) (void)hipFree(ws_);
        if (tr_) (void)hipFree(tr_);
        if (wbuf_) (void)hipFree(wbuf_);
        wbuf_ = nullptr;
        wbuf_bytes_ = 0;
        for (hipEvent_t& e : ev_)
            if (e) (void)hipEventDestroy(e);
        ws_ = tr_ = nullptr;
        for (hipEvent_t& e : ev_) e = nullptr;
    }

    smoe_geom g_{};
    smoe_weights w_{};
    smoe_hc hc_{};
    bool has_hc_ = false;
    int32_t max_tokens_ = 0;
    void* ws_ = nullptr;
    size_t ws_bytes_ = 0;
    void* tr_ = nullptr;
    size_t tr_bytes_ = 0;
    void* wbuf_ = nullptr;  // the layer's tensors, when loaded from a model
    size_t wbuf_bytes_ = 0;
    hipEvent_t ev_[SMOE_STAGE_EVENTS] = {};
};

}  // namespace smoe
