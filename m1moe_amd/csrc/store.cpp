// store.cpp — the converted model directory on disk -> HBM.
//
// Replaces WeightStore (Sources/M1MoE/WeightStore.swift: model_weights.bin
// mapped read-only, model_weights.json naming {offset, shape, dtype} per
// tensor, :15-30, :47-76, :86-116) and the per-layer expert files the
// reference preads on demand (packed_experts/layer_NN.bin,
// InferenceEngine.swift:62-77, ExpertCache.swift:49-55).  The files are the
// ones scripts/extract_olmoe.py writes (:216-266 non-expert tensors, 4-byte
// aligned; :268-345 one layer_NN.bin of E expert blocks per layer).  Here
// every expert is uploaded once (all resident in HBM) and the dense tensors
// go to the decoder; nothing is read from disk while decoding.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <vector>

#include "ctx.hpp"
#include "internal.hpp"
#include "m1moe_hip.h"

using namespace m1moe;

struct m1moe_store {
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    struct Info {
        uint64_t offset;
        int32_t dtype;
        int32_t ndim;
        int64_t shape[4];
        uint64_t bytes;
    };
    std::map<std::string, Info> tensors;
};

namespace {

// ---- a small JSON reader for the manifest: an object of objects with
// numbers, strings and arrays of numbers ------------------------------------

struct Json {
    const char* begin;
    const char* p;
    const char* end;
    std::string err;

    void ws() {
        while (p < end && std::isspace((unsigned char)*p)) ++p;
    }
    bool expect(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        char buf[64];
        snprintf(buf, sizeof buf, "expected '%c' at byte %ld", c, (long)(p - begin));
        if (err.empty()) err = buf;
        return false;
    }
    bool peek(char c) {
        ws();
        return p < end && *p == c;
    }
    bool string(std::string& out) {
        if (!expect('"')) return false;
        out.clear();
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) break;
                const char e = *p;
                out.push_back(e == 'n' ? '\n' : e == 't' ? '\t' : e);  // names are plain ASCII
            } else {
                out.push_back(*p);
            }
            ++p;
        }
        if (p >= end) {
            err = "unterminated string";
            return false;
        }
        ++p;
        return true;
    }
    bool number(double& out) {
        ws();
        char* e = nullptr;
        out = std::strtod(p, &e);
        if (e == p || e > end) {
            err = "expected a number";
            return false;
        }
        p = e;
        return true;
    }
    // skips any value (for keys the manifest does not use)
    bool skip() {
        ws();
        if (p >= end) return false;
        if (*p == '"') {
            std::string s;
            return string(s);
        }
        if (*p == '{' || *p == '[') {
            const char open = *p, close = open == '{' ? '}' : ']';
            ++p;
            if (peek(close)) return ++p, true;
            for (;;) {
                if (open == '{') {
                    std::string k;
                    if (!string(k) || !expect(':')) return false;
                }
                if (!skip()) return false;
                if (peek(',')) {
                    ++p;
                    continue;
                }
                return expect(close);
            }
        }
        if (!std::strncmp(p, "true", 4) || !std::strncmp(p, "null", 4)) return p += 4, true;
        if (!std::strncmp(p, "false", 5)) return p += 5, true;
        double d;
        return number(d);
    }
};

int32_t dtype_code(const std::string& s) {
    if (s == "bf16") return M1MOE_DT_BF16;
    if (s == "f32") return M1MOE_DT_F32;
    if (s == "u32") return M1MOE_DT_U32;
    return -1;
}

int32_t parse_manifest(const std::string& text, m1moe_store* st) {
    Json j{text.data(), text.data(), text.data() + text.size(), {}};
    if (!j.expect('{')) return fail(M1MOE_ERR_INVALID, "manifest: %s", j.err.c_str());
    if (j.peek('}')) return M1MOE_OK;
    for (;;) {
        std::string name;
        if (!j.string(name) || !j.expect(':') || !j.expect('{'))
            return fail(M1MOE_ERR_INVALID, "manifest: %s", j.err.c_str());
        m1moe_store::Info info{};
        bool has_off = false, has_shape = false, has_dtype = false;
        if (!j.peek('}')) {
            for (;;) {
                std::string key;
                if (!j.string(key) || !j.expect(':'))
                    return fail(M1MOE_ERR_INVALID, "manifest: %s", j.err.c_str());
                if (key == "offset") {
                    double d;
                    // (compared as a double before the cast: a cast of a value
                    // >= 2^64 is undefined)
                    if (!j.number(d) || !(d >= 0) || d > (double)st->size || d != (double)(uint64_t)d)
                        return fail(M1MOE_ERR_INVALID, "manifest: bad offset of %s", name.c_str());
                    info.offset = (uint64_t)d;
                    has_off = true;
                } else if (key == "shape") {
                    if (!j.expect('['))
                        return fail(M1MOE_ERR_INVALID, "manifest: bad shape of %s", name.c_str());
                    info.ndim = 0;
                    if (!j.peek(']')) {
                        for (;;) {
                            double d;
                            if (!j.number(d) || !(d >= 0) || d > 9.0e15 || info.ndim >= 4)
                                return fail(M1MOE_ERR_INVALID, "manifest: bad shape of %s", name.c_str());
                            info.shape[info.ndim++] = (int64_t)d;
                            if (j.peek(',')) {
                                ++j.p;
                                continue;
                            }
                            break;
                        }
                    }
                    if (!j.expect(']'))
                        return fail(M1MOE_ERR_INVALID, "manifest: bad shape of %s", name.c_str());
                    has_shape = true;
                } else if (key == "dtype") {
                    std::string d;
                    if (!j.string(d) || (info.dtype = dtype_code(d)) < 0)
                        return fail(M1MOE_ERR_INVALID, "manifest: dtype of %s is not bf16, f32 or u32",
                                    name.c_str());
                    has_dtype = true;
                } else if (!j.skip()) {
                    return fail(M1MOE_ERR_INVALID, "manifest: %s", j.err.c_str());
                }
                if (j.peek(',')) {
                    ++j.p;
                    continue;
                }
                break;
            }
        }
        if (!j.expect('}')) return fail(M1MOE_ERR_INVALID, "manifest: %s", j.err.c_str());
        if (!has_off || !has_shape || !has_dtype)
            return fail(M1MOE_ERR_INVALID, "manifest: %s lacks offset, shape or dtype", name.c_str());
        // element count, refused once it passes the file size (no overflow:
        // each factor is < 2^53 and the running product stays <= size)
        uint64_t n = 1;
        bool too_big = false;
        for (int d = 0; d < info.ndim; ++d) {
            const uint64_t f = (uint64_t)info.shape[d];
            if (f != 0 && n > st->size / f) too_big = true;
            else n *= f;
        }
        info.bytes = too_big ? UINT64_MAX : n * (info.dtype == M1MOE_DT_BF16 ? 2 : 4);  // TensorInfo.byteWidth, :20-27
        if (too_big || info.bytes > st->size || info.offset > st->size - info.bytes)
            return fail(M1MOE_ERR_INVALID, "manifest: %s [%llu, +%llu) lies past the end of the %llu-byte file",
                        name.c_str(), (unsigned long long)info.offset, (unsigned long long)info.bytes,
                        (unsigned long long)st->size);
        st->tensors[name] = info;
        if (j.peek(',')) {
            ++j.p;
            continue;
        }
        break;
    }
    if (!j.expect('}')) return fail(M1MOE_ERR_INVALID, "manifest: %s", j.err.c_str());
    return M1MOE_OK;
}

bool read_file(const std::string& path, std::string& out) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[1 << 16];
    size_t n;
    out.clear();
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    std::fclose(f);
    return true;
}

uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// The first `count` values of a tensor as bf16 (f32 tensors are rounded to
// nearest even: the converter keeps f32 sources as f32, scripts/
// extract_olmoe.py:243-246, while every consumer reads bf16).
int32_t tensor_bf16(m1moe_store_t st, const std::string& name, uint64_t count, std::vector<uint16_t>& out,
                    const uint16_t** direct) {
    auto it = st->tensors.find(name);
    if (it == st->tensors.end()) return fail(M1MOE_ERR_INVALID, "tensor %s is not in the manifest", name.c_str());
    const m1moe_store::Info& in = it->second;
    const uint64_t have = in.bytes / (in.dtype == M1MOE_DT_BF16 ? 2 : 4);
    if (have < count)
        return fail(M1MOE_ERR_INVALID, "tensor %s has %llu values, %llu needed", name.c_str(),
                    (unsigned long long)have, (unsigned long long)count);
    const uint8_t* src = st->base + in.offset;
    if (in.dtype == M1MOE_DT_BF16) {
        if (in.offset % 2 == 0) {
            *direct = reinterpret_cast<const uint16_t*>(src);
            return M1MOE_OK;
        }
        out.resize(count);
        std::memcpy(out.data(), src, count * 2);
    } else if (in.dtype == M1MOE_DT_F32) {
        out.resize(count);
        for (uint64_t i = 0; i < count; ++i) {
            float f;
            std::memcpy(&f, src + 4 * i, 4);
            out[i] = f32_to_bf16_rne(f);
        }
    } else {
        return fail(M1MOE_ERR_INVALID, "tensor %s is u32, a bf16 or f32 tensor was expected", name.c_str());
    }
    *direct = out.data();
    return M1MOE_OK;
}

constexpr int64_t kVec = -1;       // a vector of exactly `rows` values
constexpr int64_t kVecPrefix = -2; // a vector of at least `rows` values (the first are used)

// checks a tensor's shape against the expected [rows, cols] (or a vector)
int32_t check_shape2(m1moe_store_t st, const std::string& name, int64_t rows, int64_t cols) {
    auto it = st->tensors.find(name);
    if (it == st->tensors.end()) return fail(M1MOE_ERR_INVALID, "tensor %s is not in the manifest", name.c_str());
    const m1moe_store::Info& in = it->second;
    const bool ok = cols == kVec         ? (in.ndim == 1 && in.shape[0] == rows)
                    : cols == kVecPrefix ? (in.ndim == 1 && in.shape[0] >= rows)
                                         : (in.ndim == 2 && in.shape[0] == rows && in.shape[1] == cols);
    if (!ok)
        return fail(M1MOE_ERR_INVALID, "tensor %s has shape [%lld%s%lld], [%lld%s%lld] expected", name.c_str(),
                    (long long)in.shape[0], in.ndim > 1 ? ", " : "", in.ndim > 1 ? (long long)in.shape[1] : 0LL,
                    (long long)rows, cols < 0 ? "" : ", ", cols < 0 ? 0LL : (long long)cols);
    return M1MOE_OK;
}

int32_t upload_dense(m1moe_store_t st, m1moe_dec_t dec, int32_t which, int32_t layer, const std::string& name,
                     int64_t rows, int64_t cols) {
    int32_t rc;
    if ((rc = check_shape2(st, name, rows, cols))) return rc;
    const uint64_t count = (uint64_t)rows * (uint64_t)(cols < 0 ? 1 : cols);  // (vectors: the first rows)
    std::vector<uint16_t> tmp;
    const uint16_t* p = nullptr;
    if ((rc = tensor_bf16(st, name, count, tmp, &p))) return rc;
    return m1moe_dec_upload(dec, which, layer, p, count);
}

}  // namespace

extern "C" {

int32_t m1moe_store_open(const char* bin_path, const char* json_path, m1moe_store_t* out) {
    if (!out) return fail(M1MOE_ERR_INVALID, "out is null");
    *out = nullptr;
    if (!bin_path || !json_path) return fail(M1MOE_ERR_INVALID, "null path");
    std::string text;
    if (!read_file(json_path, text)) return fail(M1MOE_ERR_INVALID, "cannot read %s", json_path);
    m1moe_store* st = new (std::nothrow) m1moe_store;
    if (!st) return fail(M1MOE_ERR_OOM, "out of host memory");
    st->fd = ::open(bin_path, O_RDONLY);
    if (st->fd < 0) {
        delete st;
        return fail(M1MOE_ERR_INVALID, "cannot open %s", bin_path);
    }
    struct stat sb;
    if (::fstat(st->fd, &sb) != 0) {
        m1moe_store_close(st);
        return fail(M1MOE_ERR_INVALID, "cannot stat %s", bin_path);
    }
    st->size = (uint64_t)sb.st_size;
    if (st->size) {
        void* p = ::mmap(nullptr, st->size, PROT_READ, MAP_PRIVATE, st->fd, 0);  // WeightStore.swift:61
        if (p == MAP_FAILED) {
            m1moe_store_close(st);
            return fail(M1MOE_ERR_INVALID, "cannot map %s", bin_path);
        }
        st->base = static_cast<const uint8_t*>(p);
    }
    int32_t rc = parse_manifest(text, st);
    if (rc) {
        m1moe_store_close(st);
        return rc;
    }
    *out = st;
    return M1MOE_OK;
}

void m1moe_store_close(m1moe_store_t st) {
    if (!st) return;
    if (st->base) ::munmap(const_cast<uint8_t*>(st->base), st->size);
    if (st->fd >= 0) ::close(st->fd);
    delete st;
}

int32_t m1moe_store_count(m1moe_store_t st, int32_t* n) {
    if (!st || !n) return fail(M1MOE_ERR_INVALID, "null argument");
    *n = (int32_t)st->tensors.size();
    return M1MOE_OK;
}

int32_t m1moe_store_tensor(m1moe_store_t st, const char* name, const void** data, int32_t* dtype,
                           int64_t* shape, int32_t* ndim) {
    if (!st || !name) return fail(M1MOE_ERR_INVALID, "null argument");
    auto it = st->tensors.find(name);
    if (it == st->tensors.end()) return fail(M1MOE_ERR_INVALID, "tensor %s is not in the manifest", name);
    const m1moe_store::Info& in = it->second;
    if (data) *data = st->base + in.offset;
    if (dtype) *dtype = in.dtype;
    if (ndim) *ndim = in.ndim;
    if (shape)
        for (int d = 0; d < 4; ++d) shape[d] = d < in.ndim ? in.shape[d] : 0;
    return M1MOE_OK;
}

int32_t m1moe_load_model(m1moe_ctx_t ctx, m1moe_dec_t dec, const char* model_dir, int32_t threads) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!model_dir) return fail(M1MOE_ERR_INVALID, "null model_dir");
    const std::string dir(model_dir);
    const Geom& g = ctx->g;
    const uint64_t layer_bytes = (uint64_t)g.E * g.expert_bytes;

    // experts: packed_experts/layer_NN.bin, each E blocks (InferenceEngine.swift:62-77)
    std::vector<uint8_t> buf(layer_bytes);
    for (int32_t L = 0; L < g.L; ++L) {
        char name[64];
        snprintf(name, sizeof name, "/packed_experts/layer_%02d.bin", L);
        const std::string path = dir + name;
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) return fail(M1MOE_ERR_INVALID, "cannot open %s", path.c_str());
        struct stat sb;
        if (::fstat(fd, &sb) != 0 || (uint64_t)sb.st_size != layer_bytes) {
            ::close(fd);
            return fail(M1MOE_ERR_INVALID, "%s: %lld bytes, %d experts x %llu expected", path.c_str(),
                        (long long)sb.st_size, g.E, (unsigned long long)g.expert_bytes);
        }
        // parallel preads of contiguous ranges
        const int nt = threads < 1 ? 1 : (threads > 32 ? 32 : threads);
        std::vector<std::thread> pool;
        std::vector<int> ok(nt, 1);
        for (int t = 0; t < nt; ++t)
            pool.emplace_back([&, t]() {
                uint64_t a = layer_bytes * t / nt, b = layer_bytes * (t + 1) / nt;
                while (a < b) {
                    const ssize_t r = ::pread(fd, buf.data() + a, b - a, (off_t)a);
                    if (r <= 0) {
                        ok[t] = 0;
                        return;
                    }
                    a += (uint64_t)r;
                }
            });
        for (auto& th : pool) th.join();
        ::close(fd);
        for (int t = 0; t < nt; ++t)
            if (!ok[t]) return fail(M1MOE_ERR_INVALID, "short read of %s", path.c_str());
        if ((rc = m1moe_upload_layer_experts(ctx, L, buf.data(), layer_bytes))) return rc;
    }

    m1moe_store_t st = nullptr;
    if ((rc = m1moe_store_open((dir + "/model_weights.bin").c_str(), (dir + "/model_weights.json").c_str(), &st)))
        return rc;
    struct Closer {
        m1moe_store_t s;
        ~Closer() { m1moe_store_close(s); }
    } closer{st};

    // routers (WeightKeys.router, InferenceEngine.swift:593-598: OLMoE mlp.gate,
    // Mixtral block_sparse_moe.gate)
    for (int32_t L = 0; L < g.L; ++L) {
        std::string name = "model.layers." + std::to_string(L) + ".mlp.gate.weight";
        if (!st->tensors.count(name)) name = "model.layers." + std::to_string(L) + ".block_sparse_moe.gate.weight";
        if ((rc = check_shape2(st, name, g.E, g.h))) return rc;
        std::vector<uint16_t> tmp;
        const uint16_t* p = nullptr;
        if ((rc = tensor_bf16(st, name, (uint64_t)g.E * g.h, tmp, &p))) return rc;
        if ((rc = m1moe_upload_router(ctx, L, p, (uint64_t)g.E * g.h))) return rc;
    }
    if (!dec) return M1MOE_OK;

    // dense tensors (WeightKeys, InferenceEngine.swift:580-599)
    int32_t V, nh, nkv, hd, qkn;
    if ((rc = dec_dims(dec, &V, &nh, &nkv, &hd, &qkn))) return rc;
    const int64_t h = g.h, qd = (int64_t)nh * hd, kvd = (int64_t)nkv * hd;
    if ((rc = upload_dense(st, dec, M1MOE_W_EMBED, 0, "model.embed_tokens.weight", V, h)) ||
        (rc = upload_dense(st, dec, M1MOE_W_LM_HEAD, 0, "lm_head.weight", V, h)) ||
        (rc = upload_dense(st, dec, M1MOE_W_FINAL_NORM, 0, "model.norm.weight", h, kVec)))
        return rc;
    for (int32_t L = 0; L < g.L; ++L) {
        const std::string pre = "model.layers." + std::to_string(L) + ".";
        if ((rc = upload_dense(st, dec, M1MOE_W_IN_NORM, L, pre + "input_layernorm.weight", h, kVec)) ||
            (rc = upload_dense(st, dec, M1MOE_W_POST_NORM, L, pre + "post_attention_layernorm.weight", h, kVec)) ||
            (rc = upload_dense(st, dec, M1MOE_W_Q, L, pre + "self_attn.q_proj.weight", qd, h)) ||
            (rc = upload_dense(st, dec, M1MOE_W_K, L, pre + "self_attn.k_proj.weight", kvd, h)) ||
            (rc = upload_dense(st, dec, M1MOE_W_V, L, pre + "self_attn.v_proj.weight", kvd, h)) ||
            (rc = upload_dense(st, dec, M1MOE_W_O, L, pre + "self_attn.o_proj.weight", h, qd)))
            return rc;
        if (qkn) {
            // the reference reads the first head_dim values and applies them to
            // every head (InferenceEngine.swift:199-208, 538-548)
            if ((rc = upload_dense(st, dec, M1MOE_W_Q_NORM, L, pre + "self_attn.q_norm.weight", hd, kVecPrefix)) ||
                (rc = upload_dense(st, dec, M1MOE_W_K_NORM, L, pre + "self_attn.k_norm.weight", hd, kVecPrefix)))
                return rc;
        }
    }
    return M1MOE_OK;
}

}  // extern "C"
