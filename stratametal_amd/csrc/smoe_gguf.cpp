// stratametal_amd/csrc/smoe_gguf.cpp - GGUF v3 models on the host (the reader: mapping, metadata, tensor directory;
// split models; tensors by name) and the loader of one layer's MoE tensors into device memory.
//
// The reader follows the GGUF v3 file format as the reference reads it (include/strata/artifact/gguf_reader.hpp:
// 340-476: header, every metadata value type including arrays, the tensor directory, the data section at the
// file's alignment; a duplicate tensor name refuses the file) and the reference's split models
// (include/strata/artifact/gguf_split.hpp, gguf_reader.hpp:500-566: `<stem>-NNNNN-of-MMMMM.gguf`, the metadata in
// shard 1, split.count / split.no / split.tensors.count agreeing, no tensor in two shards).  The layer loader is the
// tensor side of FfnExec::load (metal/src/layer_exec.cpp:369-431; expert_spans, metal/src/layer_exec.cpp:109-123):
// blk.<L>.ffn_{gate,up,down}_exps, ffn_gate_inp, the shared expert's planes and gate, and the hyper-connection
// tensors, each into a 256-byte aligned slot of one device buffer the caller provides.
#include "smoe.h"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace smoe {
smoe_status report(smoe_status s, const std::string& why);  // smoe_api.cpp: the thread's last error
}

namespace {

using smoe::report;

enum : uint32_t { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64 };

struct MetaValue {
    uint32_t type = 0;
    uint64_t u = 0;      // integer and bool values (signed ones sign-extended)
    double f = 0.0;      // float values
    std::string s;       // string values
    uint32_t elem = 0;   // arrays: element type and count (elements are skipped)
    uint64_t count = 0;
};

struct TensorDesc {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};  // GGUF order: ne[0] varies fastest (a row)
    uint32_t type = 0;
    uint64_t offset = 0;            // from the data section
};

// Values and bytes per block of the GGUF element and block formats this library knows.
bool type_blocks(uint32_t t, uint64_t& qk, uint64_t& bytes) {
    static const struct { uint32_t t, qk, bytes; } kTab[] = {
        {0, 1, 4},      {1, 1, 2},      {30, 1, 2},     {24, 1, 1},     {25, 1, 2},   {26, 1, 4},   {27, 1, 8},
        {28, 1, 8},     {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},  {8, 32, 34},  {9, 32, 36},
        {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292},
        {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},  {20, 32, 18}, {21, 256, 110},
        {22, 256, 82},  {23, 256, 136}, {29, 256, 56},  {42, 64, 18}};
    for (const auto& e : kTab)
        if (e.t == t) {
            qk = e.qk;
            bytes = e.bytes;
            return true;
        }
    return false;
}

// Payload bytes from the shape; 0 for an unknown type, a row that is not whole blocks, or an overflow.
uint64_t payload_bytes(const TensorDesc& t) {
    uint64_t qk = 0, bb = 0;
    if (!type_blocks(t.type, qk, bb) || t.n_dims == 0 || t.ne[0] % qk) return 0;
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
        if (t.ne[d] == 0 || n > std::numeric_limits<uint64_t>::max() / t.ne[d]) return 0;
        n *= t.ne[d];
    }
    const uint64_t blocks = n / qk;
    return blocks > std::numeric_limits<uint64_t>::max() / bb ? 0 : blocks * bb;
}

// Bounds-checked little-endian reads over the mapped header.
class Cursor {
   public:
    Cursor(const uint8_t* b, uint64_t n) : b_(b), n_(n) {}
    template <class V>
    V get() {
        need(sizeof(V));
        V v;
        std::memcpy(&v, b_ + p_, sizeof(V));
        p_ += sizeof(V);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (len > (1u << 30)) throw std::runtime_error("GGUF: implausible string length");
        need(len);
        std::string s(reinterpret_cast<const char*>(b_ + p_), (size_t)len);
        p_ += len;
        return s;
    }
    uint64_t pos() const { return p_; }

   private:
    void need(uint64_t k) const {
        if (k > n_ || p_ > n_ - k) throw std::runtime_error("GGUF: the header ends before its contents");
    }
    const uint8_t* b_;
    uint64_t n_, p_ = 0;
};

MetaValue read_value(Cursor& c, uint32_t type, int depth) {
    if (depth > 2) throw std::runtime_error("GGUF: nested metadata arrays");
    MetaValue v;
    v.type = type;
    switch (type) {
        case kU8: v.u = c.get<uint8_t>(); break;
        case kI8: v.u = (uint64_t)(int64_t)c.get<int8_t>(); break;
        case kU16: v.u = c.get<uint16_t>(); break;
        case kI16: v.u = (uint64_t)(int64_t)c.get<int16_t>(); break;
        case kU32: v.u = c.get<uint32_t>(); break;
        case kI32: v.u = (uint64_t)(int64_t)c.get<int32_t>(); break;
        case kU64: v.u = c.get<uint64_t>(); break;
        case kI64: v.u = (uint64_t)c.get<int64_t>(); break;
        case kBool: v.u = c.get<uint8_t>() ? 1 : 0; break;
        case kF32: v.f = c.get<float>(); break;
        case kF64: v.f = c.get<double>(); break;
        case kString: v.s = c.str(); break;
        case kArray:
            v.elem = c.get<uint32_t>();
            v.count = c.get<uint64_t>();
            if (v.count > (1u << 24)) throw std::runtime_error("GGUF: implausible array length");
            for (uint64_t i = 0; i < v.count; ++i) read_value(c, v.elem, depth + 1);
            break;
        default: throw std::runtime_error("GGUF: unknown metadata value type " + std::to_string(type));
    }
    return v;
}

struct Shard {
    std::string path;
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t size = 0, data_start = 0, alignment = 32;
    uint32_t version = 0;
    std::map<std::string, MetaValue> meta;
    std::vector<TensorDesc> tensors;

    explicit Shard(const std::string& p) : path(p) {
        try {  // a refused file releases its descriptor and mapping here: the destructor does not run
            fd = ::open(p.c_str(), O_RDONLY);
            if (fd < 0) throw std::runtime_error("cannot open " + p);
            struct stat st {};
            if (fstat(fd, &st) != 0) throw std::runtime_error("cannot stat " + p);
            size = (uint64_t)st.st_size;
            if (size < 24) throw std::runtime_error("GGUF: " + p + " is too short for a header");
            void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (m == MAP_FAILED) throw std::runtime_error("cannot map " + p);
            base = static_cast<const uint8_t*>(m);
            parse();
        } catch (...) {
            release();
            throw;
        }
    }
    ~Shard() { release(); }
    Shard(const Shard&) = delete;
    Shard& operator=(const Shard&) = delete;

    const MetaValue* get(const std::string& k) const {
        const auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second;
    }

   private:
    void release() {
        if (base) munmap(const_cast<uint8_t*>(base), size);
        if (fd >= 0) ::close(fd);
        base = nullptr;
        fd = -1;
    }
    void parse() {
        Cursor c(base, size);
        if (c.get<uint32_t>() != 0x46554747u) throw std::runtime_error("GGUF: " + path + " has no GGUF magic");
        version = c.get<uint32_t>();
        if (version != 3) throw std::runtime_error("GGUF: " + path + " is v" + std::to_string(version) + ", v3 is read");
        const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
        if (n_tensors > (1u << 24) || n_kv > (1u << 24)) throw std::runtime_error("GGUF: implausible header counts");
        for (uint64_t i = 0; i < n_kv; ++i) {
            std::string k = c.str();
            const uint32_t t = c.get<uint32_t>();
            MetaValue v = read_value(c, t, 0);
            meta.emplace(std::move(k), std::move(v));  // a repeated key keeps its first value, as the reference's map does
        }
        std::map<std::string, int> seen;
        tensors.resize((size_t)n_tensors);
        for (auto& t : tensors) {
            t.name = c.str();
            if (!seen.emplace(t.name, 0).second)
                throw std::runtime_error("GGUF: tensor '" + t.name + "' is listed twice in " + path);
            t.n_dims = c.get<uint32_t>();
            if (t.n_dims == 0 || t.n_dims > 4) throw std::runtime_error("GGUF: tensor '" + t.name + "' has a bad rank");
            for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = c.get<uint64_t>();
            t.type = c.get<uint32_t>();
            t.offset = c.get<uint64_t>();
        }
        if (const MetaValue* a = get("general.alignment"); a && a->u) alignment = a->u;
        // an alignment beyond the file puts the data section past its end (and keeps the rounding below from
        // wrapping around)
        if (alignment > size) throw std::runtime_error("GGUF: " + path + ": the data section starts past the end");
        data_start = (c.pos() + alignment - 1) / alignment * alignment;
        if (data_start > size) throw std::runtime_error("GGUF: " + path + ": the data section starts past the end");
    }
};

// The shard paths of the model `any` belongs to: `<stem>-NNNNN-of-MMMMM.gguf` names M shards; anything else is a
// model of one file.
std::vector<std::string> shard_paths(const std::string& any) {
    const size_t at = any.rfind("-of-");
    auto digits = [&](size_t from) {
        int v = 0;
        for (size_t i = 0; i < 5; ++i) {
            const char ch = any[from + i];
            if (ch < '0' || ch > '9') return -1;
            v = v * 10 + (ch - '0');
        }
        return v;
    };
    if (at == std::string::npos || at < 6 || any[at - 6] != '-' || any.size() != at + 4 + 5 + 5 ||
        any.compare(at + 9, 5, ".gguf") != 0)
        return {any};
    const int no = digits(at - 5), n = digits(at + 4);
    if (no < 1 || n < 1 || no > n) return {any};
    std::vector<std::string> out;
    for (int i = 1; i <= n; ++i) {
        char num[8];
        std::snprintf(num, sizeof num, "%05d", i);
        std::string p = any;
        p.replace(at - 5, 5, num);
        out.push_back(p);
    }
    return out;
}

}  // namespace

struct smoe_model {
    std::vector<std::unique_ptr<Shard>> shards;
    std::map<std::string, std::pair<int, const TensorDesc*>> index;
    std::vector<std::pair<int, const TensorDesc*>> order;  // every tensor, shard by shard

    explicit smoe_model(const std::string& any) {
        const std::vector<std::string> paths = shard_paths(any);
        for (const auto& p : paths) {
            struct stat st {};
            if (::stat(p.c_str(), &st) != 0)
                throw std::runtime_error("model shard " + p + " is missing (" + std::to_string(shards.size() + 1) +
                                         " of " + std::to_string(paths.size()) + ")");
            shards.push_back(std::make_unique<Shard>(p));
        }
        validate_split();
        for (size_t i = 0; i < shards.size(); ++i)
            for (const auto& t : shards[i]->tensors) {
                const auto ins = index.emplace(t.name, std::make_pair((int)i, &t));
                if (!ins.second)
                    throw std::runtime_error("GGUF: tensor " + t.name + " is in two shards (" +
                                             shards[ins.first->second.first]->path + " and " + shards[i]->path + ")");
                order.emplace_back((int)i, &t);
            }
    }

   private:
    void validate_split() const {
        const size_t n = shards.size();
        const MetaValue* c0 = shards[0]->get("split.count");
        if (n == 1) {
            if (c0 && c0->u > 1)
                throw std::runtime_error("GGUF: " + shards[0]->path + " is shard 1 of " + std::to_string(c0->u) +
                                         ", opened as a whole model");
            return;
        }
        if (!shards[0]->get("general.architecture"))
            throw std::runtime_error("GGUF: " + shards[0]->path + " carries no general.architecture (the metadata shard)");
        const MetaValue* total = shards[0]->get("split.tensors.count");
        uint64_t sum = 0;
        for (size_t i = 0; i < n; ++i) {
            const Shard& s = *shards[i];
            const MetaValue *cnt = s.get("split.count"), *no = s.get("split.no"), *tc = s.get("split.tensors.count");
            if (!cnt || !no || cnt->u != n || no->u != i || (total && (!tc || tc->u != total->u)))
                throw std::runtime_error("GGUF: " + s.path + " does not declare itself shard " + std::to_string(i + 1) +
                                         " of " + std::to_string(n) + " of this model (split.count / split.no / "
                                         "split.tensors.count)");
            sum += s.tensors.size();
        }
        if (total && sum != total->u)
            throw std::runtime_error("GGUF: the shards hold " + std::to_string(sum) + " tensors, split.tensors.count says " +
                                     std::to_string(total->u));
    }
};

namespace {

smoe_status describe(const smoe_model* m, int shard, const TensorDesc& t, smoe_tensor_info* info) {
    const Shard& s = *m->shards[(size_t)shard];
    const uint64_t bytes = payload_bytes(t), payload = s.size - s.data_start;
    if (bytes == 0)
        return report(SMOE_ETYPE, "tensor " + t.name + ": type " + std::to_string(t.type) +
                                      " has no known block size here, or its rows are not whole blocks");
    if (t.offset > payload || bytes > payload - t.offset)
        return report(SMOE_ESIZE, "tensor " + t.name + " does not fit inside " + s.path);
    if (info) {
        std::memset(info, 0, sizeof *info);
        info->type = (int32_t)t.type;
        info->n_dims = (int32_t)t.n_dims;
        info->shard = shard;
        for (int d = 0; d < 4; ++d) info->ne[d] = t.ne[d];
        info->bytes = bytes;
        info->file_offset = s.data_start + t.offset;
        info->host = s.base + s.data_start + t.offset;
    }
    return SMOE_OK;
}

const TensorDesc* lookup(const smoe_model* m, const std::string& name, int* shard) {
    const auto it = m->index.find(name);
    if (it == m->index.end()) return nullptr;
    *shard = it->second.first;
    return it->second.second;
}

std::string layer_name(int layer, const char* suffix) { return "blk." + std::to_string(layer) + "." + suffix; }

constexpr int kGgufF32 = 0, kGgufF16 = 1, kGgufBf16 = 30;

// A type the block's q8_1 GEMV contract runs for a shared projection: Q2_0, IQ2_S and the native types of smoe.h.
bool gemv_type(uint32_t t) {
    switch (t) {
        case SMOE_Q2_0: case SMOE_IQ2_S: case SMOE_Q8_0: case SMOE_Q4_0: case SMOE_Q5_0: case SMOE_IQ4_NL:
        case SMOE_IQ4_XS: case SMOE_Q3_K: case SMOE_Q4_K: case SMOE_Q5_K: case SMOE_Q6_K:
            return true;
        default:
            return false;
    }
}

// One tensor of the layer, resolved and checked (type, shape), or a refusal.
struct Part {
    const TensorDesc* t = nullptr;
    int shard = 0;
    smoe_tensor_info info{};
};
smoe_status find_part(const smoe_model* m, int layer, const char* suffix, bool required, Part& p) {
    const std::string name = layer_name(layer, suffix);
    p.t = lookup(m, name, &p.shard);
    if (!p.t) return required ? report(SMOE_EINVAL, "layer " + std::to_string(layer) + " has no " + name) : SMOE_OK;
    return describe(m, p.shard, *p.t, &p.info);
}

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

struct LayerParts {
    Part gate, up, down, router, gsh, ush, dsh, ginp, hdown, hup, hinj, hnorm;
};

// The plan of a layer: its tensors, geometry and device slots.
smoe_status plan_layer(const smoe_model* m, int layer, int top_k, int with_shared, LayerParts& P, smoe_layer_plan* out) {
    smoe_status s;
    if ((s = find_part(m, layer, "ffn_gate_exps.weight", true, P.gate)) != SMOE_OK) return s;
    if ((s = find_part(m, layer, "ffn_up_exps.weight", true, P.up)) != SMOE_OK) return s;
    if ((s = find_part(m, layer, "ffn_down_exps.weight", true, P.down)) != SMOE_OK) return s;
    if ((s = find_part(m, layer, "ffn_gate_inp.weight", true, P.router)) != SMOE_OK) return s;
    const uint64_t H = P.gate.t->ne[0], F = P.gate.t->ne[1], E = P.gate.t->ne[2];
    // every dimension is narrowed to int32 below: refuse what would not survive it
    constexpr uint64_t kDimMax = 0x7FFFFFFFu;
    if (H > kDimMax || F > kDimMax || E > kDimMax)
        return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": ffn_gate_exps has a dimension beyond int32");
    auto shape = [&](const Part& p, uint64_t a, uint64_t b, uint64_t c, const char* what) -> smoe_status {
        if (p.t->ne[0] != a || p.t->ne[1] != b || p.t->ne[2] != c || p.t->ne[3] != 1)
            return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": " + p.t->name + " has not the shape of " +
                                           what);
        return SMOE_OK;
    };
    if ((s = shape(P.up, H, F, E, "ffn_gate_exps")) != SMOE_OK) return s;
    if ((s = shape(P.down, F, H, E, "[n_ff][n_embd][n_expert]")) != SMOE_OK) return s;
    if ((s = shape(P.router, H, E, 1, "[n_embd][n_expert]")) != SMOE_OK) return s;
    if (P.gate.t->type != P.up.t->type || P.gate.t->type != P.down.t->type)
        return report(SMOE_ETYPE, "layer " + std::to_string(layer) + ": the routed gate, up and down planes are of "
                                                                     "different types");
    if (P.router.t->type != kGgufBf16 && P.router.t->type != kGgufF32)
        return report(SMOE_ETYPE, "layer " + std::to_string(layer) + ": ffn_gate_inp is neither BF16 nor F32");
    std::memset(out, 0, sizeof *out);
    smoe_geom& g = out->geom;
    g.n_embd = (int32_t)H;
    g.n_ff = (int32_t)F;
    g.n_expert = (int32_t)E;
    g.w_type = (int32_t)P.gate.t->type;
    g.router_dtype = P.router.t->type == kGgufF32 ? SMOE_ROUTER_F32 : SMOE_ROUTER_BF16;
    g.sh_type = -1;
    if (top_k <= 0) {  // the model's own expert_used_count
        const MetaValue* arch = m->shards[0]->get("general.architecture");
        const MetaValue* ku = arch ? m->shards[0]->get(arch->s + ".expert_used_count") : nullptr;
        if (!ku) return report(SMOE_EINVAL, "no top_k given and the model declares no <architecture>.expert_used_count");
        if (ku->u > 64) return report(SMOE_EINVAL, "<architecture>.expert_used_count is beyond 64");
        top_k = (int)ku->u;
    }
    g.top_k = top_k;
    if (with_shared) {
        if ((s = find_part(m, layer, "ffn_gate_shexp.weight", true, P.gsh)) != SMOE_OK) return s;
        if ((s = find_part(m, layer, "ffn_up_shexp.weight", true, P.ush)) != SMOE_OK) return s;
        if ((s = find_part(m, layer, "ffn_down_shexp.weight", true, P.dsh)) != SMOE_OK) return s;
        if ((s = find_part(m, layer, "ffn_gate_inp_shexp.weight", true, P.ginp)) != SMOE_OK) return s;
        const uint64_t Fs = P.gsh.t->ne[1];
        if (Fs > kDimMax)
            return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": ffn_gate_shexp has a dimension beyond int32");
        // each shared projection must be a type the block's GEMV contract implements: smoe_geom reads a zero
        // projection type as "the shared expert's type", so GGML type 0 (F32) must not reach it
        for (const Part* q : {&P.gsh, &P.ush, &P.dsh})
            if (!gemv_type(q->t->type))
                return report(SMOE_ETYPE, "layer " + std::to_string(layer) + ": " + q->t->name + " is of GGML type " +
                                              std::to_string(q->t->type) + ", which the shared expert does not run");
        if ((s = shape(P.gsh, H, Fs, 1, "[n_embd][n_ff_shared]")) != SMOE_OK) return s;
        if ((s = shape(P.ush, H, Fs, 1, "[n_embd][n_ff_shared]")) != SMOE_OK) return s;
        if ((s = shape(P.dsh, Fs, H, 1, "[n_ff_shared][n_embd]")) != SMOE_OK) return s;
        if (P.ginp.t->ne[0] != H || P.ginp.t->ne[1] != 1 || P.ginp.t->ne[2] != 1)
            return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": ffn_gate_inp_shexp is not [n_embd]");
        if (P.ginp.t->type != kGgufBf16 && P.ginp.t->type != kGgufF32)
            return report(SMOE_ETYPE, "layer " + std::to_string(layer) + ": ffn_gate_inp_shexp is neither BF16 nor F32");
        g.n_ff_shared = (int32_t)Fs;
        g.sh_type = (int32_t)P.gsh.t->type;
        g.sh_gate_type = (int32_t)P.gsh.t->type;
        g.sh_up_type = (int32_t)P.ush.t->type;
        g.sh_down_type = (int32_t)P.dsh.t->type;
    }
    // the hyper-connection tensors: all four, or none
    if ((s = find_part(m, layer, "hc_ffn_down.weight", false, P.hdown)) != SMOE_OK) return s;
    if ((s = find_part(m, layer, "hc_ffn_up.weight", false, P.hup)) != SMOE_OK) return s;
    if ((s = find_part(m, layer, "hc_ffn_inject.weight", false, P.hinj)) != SMOE_OK) return s;
    if ((s = find_part(m, layer, "hc_ffn_norm.weight", false, P.hnorm)) != SMOE_OK) return s;
    const int n_hc = (P.hdown.t ? 1 : 0) + (P.hup.t ? 1 : 0) + (P.hinj.t ? 1 : 0) + (P.hnorm.t ? 1 : 0);
    if (n_hc != 0 && n_hc != 4)
        return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": only some of the hc_ffn tensors are present");
    if (n_hc == 4) {
        const uint64_t hc = P.hinj.t->ne[1], lr = P.hdown.t->ne[1];
        if (hc == 0 || hc > 64 || lr == 0 || lr > 65536)  // bounds that keep the products below exact
            return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": implausible hc_ffn stream counts");
        if (P.hdown.t->type != kGgufBf16 || P.hup.t->type != kGgufBf16 || P.hinj.t->type != kGgufBf16 ||
            P.hnorm.t->type != kGgufF32)
            return report(SMOE_ETYPE, "layer " + std::to_string(layer) + ": hc_ffn_{down,up,inject} must be BF16 and "
                                                                         "hc_ffn_norm F32");
        const uint64_t nrm = P.hnorm.t->ne[0] * P.hnorm.t->ne[1] * P.hnorm.t->ne[2];
        if (P.hdown.t->ne[0] != hc * H || P.hup.t->ne[0] != lr || P.hup.t->ne[1] != hc * H ||
            P.hinj.t->ne[0] != hc * H || nrm != hc * H)
            return report(SMOE_EINVAL, "layer " + std::to_string(layer) + ": the hc_ffn tensors' shapes disagree");
        out->hc.hc = (int32_t)hc;
        out->hc.hc_lr = (int32_t)lr;
        out->hc.eps = 1e-6f;  // FfnExec::run's gated-residual epsilon
    }
    // device slots, each 256-byte aligned, in this order
    size_t o = 0;
    auto take = [&](uint64_t b) { const size_t at = o; o = up256(o + (size_t)b); return at; };
    out->off[0] = take(P.gate.info.bytes);
    out->off[1] = take(P.up.info.bytes);
    out->off[2] = take(P.down.info.bytes);
    out->off[3] = take(P.router.info.bytes);
    if (with_shared) {
        out->off[4] = take(P.gsh.info.bytes);
        out->off[5] = take(P.ush.info.bytes);
        out->off[6] = take(P.dsh.info.bytes);
        out->off[7] = take(H * 2);  // the shared gate as bf16
    }
    if (n_hc == 4) {
        out->off[8] = take(P.hnorm.info.bytes);
        out->off[9] = take(P.hdown.info.bytes);
        out->off[10] = take(P.hup.info.bytes);
        out->off[11] = take(P.hinj.info.bytes);
    }
    out->device_bytes = o;
    out->layer = layer;
    out->with_shared = with_shared ? 1 : 0;
    // the block itself must accept the geometry
    if (smoe_workspace_bytes(&out->geom, 1) == 0) return SMOE_EINVAL;  // the reason is the library's last error
    return SMOE_OK;
}

uint16_t bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 64u);  // NaN, quieted
    return (uint16_t)((u + ((u >> 16) & 1u) + 0x7FFFu) >> 16);
}

}  // namespace

extern "C" {

smoe_status smoe_model_open(const char* path, smoe_model** out) {
    if (!path || !out) return report(SMOE_ENULL, "model_open: NULL path or handle");
    *out = nullptr;
    try {
        *out = new smoe_model(path);
    } catch (const std::exception& e) {
        return report(SMOE_EINVAL, e.what());
    }
    return report(SMOE_OK, "");
}

void smoe_model_close(smoe_model* m) { delete m; }

int32_t smoe_model_n_shards(const smoe_model* m) { return m ? (int32_t)m->shards.size() : 0; }

int64_t smoe_model_n_tensors(const smoe_model* m) { return m ? (int64_t)m->order.size() : 0; }

smoe_status smoe_model_tensor(const smoe_model* m, const char* name, smoe_tensor_info* info) {
    if (!m || !name) return report(SMOE_ENULL, "model_tensor: NULL model or name");
    int shard = 0;
    const TensorDesc* t = lookup(m, name, &shard);
    if (!t) return report(SMOE_EINVAL, std::string("model has no tensor ") + name);
    const smoe_status s = describe(m, shard, *t, info);
    return s == SMOE_OK ? report(SMOE_OK, "") : s;
}

smoe_status smoe_model_tensor_at(const smoe_model* m, int64_t i, char* name, size_t name_cap, smoe_tensor_info* info) {
    if (!m) return report(SMOE_ENULL, "model_tensor_at: NULL model");
    if (i < 0 || i >= (int64_t)m->order.size()) return report(SMOE_EINVAL, "model_tensor_at: index out of range");
    const auto& e = m->order[(size_t)i];
    if (name) {
        if (name_cap < e.second->name.size() + 1) return report(SMOE_ESIZE, "model_tensor_at: name buffer too small");
        std::memcpy(name, e.second->name.c_str(), e.second->name.size() + 1);
    }
    const smoe_status s = describe(m, e.first, *e.second, info);
    return s == SMOE_OK ? report(SMOE_OK, "") : s;
}

smoe_status smoe_model_meta_u64(const smoe_model* m, const char* key, uint64_t* value) {
    if (!m || !key || !value) return report(SMOE_ENULL, "model_meta_u64: NULL argument");
    const MetaValue* v = m->shards[0]->get(key);
    if (!v) return report(SMOE_EINVAL, std::string("no metadata key ") + key);
    if (v->type == kArray) {
        *value = v->count;  // an array's element count
    } else if (v->type == kString || v->type == kF32 || v->type == kF64) {
        return report(SMOE_ETYPE, std::string("metadata ") + key + " is not an integer");
    } else {
        *value = v->u;
    }
    return report(SMOE_OK, "");
}

smoe_status smoe_model_meta_str(const smoe_model* m, const char* key, char* buf, size_t cap) {
    if (!m || !key || !buf) return report(SMOE_ENULL, "model_meta_str: NULL argument");
    const MetaValue* v = m->shards[0]->get(key);
    if (!v) return report(SMOE_EINVAL, std::string("no metadata key ") + key);
    if (v->type != kString) return report(SMOE_ETYPE, std::string("metadata ") + key + " is not a string");
    if (cap < v->s.size() + 1) return report(SMOE_ESIZE, std::string("metadata ") + key + ": buffer too small");
    std::memcpy(buf, v->s.c_str(), v->s.size() + 1);
    return report(SMOE_OK, "");
}

smoe_status smoe_layer_plan_for(const smoe_model* m, int32_t layer, int32_t top_k, int32_t with_shared,
                                smoe_layer_plan* plan) {
    if (!m || !plan) return report(SMOE_ENULL, "layer_plan: NULL model or plan");
    LayerParts P;
    const smoe_status s = plan_layer(m, layer, top_k, with_shared, P, plan);
    return s == SMOE_OK ? report(SMOE_OK, "") : s;
}

smoe_status smoe_layer_upload(const smoe_model* m, const smoe_layer_plan* plan, void* device, size_t device_bytes,
                              smoe_weights* w, smoe_hc* hc, void* hip_stream) {
    if (!m || !plan || !w) return report(SMOE_ENULL, "layer_upload: NULL model, plan or weights");
    LayerParts P;
    smoe_layer_plan again;
    smoe_status s = plan_layer(m, plan->layer, plan->geom.top_k, plan->with_shared, P, &again);
    if (s != SMOE_OK) return s;
    if (std::memcmp(&again.off, &plan->off, sizeof again.off) != 0 || again.device_bytes != plan->device_bytes)
        return report(SMOE_EINVAL, "layer_upload: the plan is not this model's plan of this layer");
    if (!device) return report(SMOE_ENULL, "layer_upload: NULL device buffer");
    if (((uintptr_t)device & 255) != 0) return report(SMOE_EALIGN, "layer_upload: the device buffer must be 256-byte aligned");
    if (device_bytes < plan->device_bytes)
        return report(SMOE_ESIZE, "layer_upload: the device buffer holds " + std::to_string(device_bytes) + " bytes, the "
                                  "layer needs " + std::to_string(plan->device_bytes));
    if (hc && plan->hc.hc == 0) return report(SMOE_EINVAL, "layer_upload: the layer has no hc_ffn tensors");
    hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
    uint8_t* d = static_cast<uint8_t*>(device);
    std::vector<uint16_t> ginp;
    auto copy = [&](const Part& p, size_t off) -> hipError_t {
        return hipMemcpyAsync(d + off, p.info.host, (size_t)p.info.bytes, hipMemcpyHostToDevice, st);
    };
    hipError_t e = hipSuccess;
    const size_t* off = plan->off;
    for (const auto& [p, o] : {std::pair<const Part*, size_t>{&P.gate, off[0]}, {&P.up, off[1]}, {&P.down, off[2]},
                               {&P.router, off[3]}})
        if (e == hipSuccess) e = copy(*p, o);
    if (plan->with_shared && e == hipSuccess) {
        e = copy(P.gsh, off[4]);
        if (e == hipSuccess) e = copy(P.ush, off[5]);
        if (e == hipSuccess) e = copy(P.dsh, off[6]);
        if (e == hipSuccess) {
            const int64_t H = plan->geom.n_embd;
            if (P.ginp.t->type == kGgufBf16) {
                e = hipMemcpyAsync(d + off[7], P.ginp.info.host, (size_t)H * 2, hipMemcpyHostToDevice, st);
            } else {  // F32 stored: the block's contract takes the shared gate as bf16 (RNE)
                ginp.resize((size_t)H);
                const float* src = static_cast<const float*>(P.ginp.info.host);
                for (int64_t i = 0; i < H; ++i) ginp[(size_t)i] = bf16_rne(src[i]);
                e = hipMemcpyAsync(d + off[7], ginp.data(), (size_t)H * 2, hipMemcpyHostToDevice, st);
            }
        }
    }
    if (hc && e == hipSuccess) {
        e = copy(P.hnorm, off[8]);
        if (e == hipSuccess) e = copy(P.hdown, off[9]);
        if (e == hipSuccess) e = copy(P.hup, off[10]);
        if (e == hipSuccess) e = copy(P.hinj, off[11]);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);  // the host sources (the mapping, the converted gate) are read
    if (e != hipSuccess) return report(SMOE_EDEVICE, std::string("layer_upload: ") + hipGetErrorString(e));
    std::memset(w, 0, sizeof *w);
    w->gate_exps = d + off[0];
    w->up_exps = d + off[1];
    w->down_exps = d + off[2];
    w->router = d + off[3];
    if (plan->with_shared) {
        w->gate_sh = d + off[4];
        w->up_sh = d + off[5];
        w->down_sh = d + off[6];
        w->gate_inp_sh = reinterpret_cast<const uint16_t*>(d + off[7]);
    }
    if (hc) {
        *hc = plan->hc;
        hc->norm = reinterpret_cast<const float*>(d + off[8]);
        hc->down = reinterpret_cast<const uint16_t*>(d + off[9]);
        hc->up = reinterpret_cast<const uint16_t*>(d + off[10]);
        hc->inject = reinterpret_cast<const uint16_t*>(d + off[11]);
    }
    return report(SMOE_OK, "");
}

}  // extern "C"
