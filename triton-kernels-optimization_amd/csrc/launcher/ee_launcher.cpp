// ee_launcher.cpp -- host side of the C ABI in include/entropy_engine.h.
//
// Loads the gfx950 code objects named by entropy_engine_meta.json with
// hipModuleLoadData, resolves every kernel with hipModuleGetFunction, checks
// the launch geometry the meta declares against the functions' attributes,
// and launches with hipModuleLaunchKernel on the caller's stream.  Every
// argument check happens before the first HIP call of an entry point.
// Role of the reference's CubinEngine (EE/csrc/engine.cpp:23-216); the
// meta-JSON reader serves the same purpose as its from_metadata
// (engine.cpp:168-199), on a real JSON parser.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "../common/ee_kernel_args.h"
#include "entropy_engine.h"

#define EE_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define EE_HIP(call, what)                                                                   \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess) return fail(EE_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e_)); \
    } while (0)

// ---------------------------------------------------------------- JSON reader
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;
    const Json* get(const std::string& k) const {
        if (kind != OBJ) return nullptr;
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
};

struct JsonParser {
    const std::string& s;
    size_t i = 0;
    std::string err;
    explicit JsonParser(const std::string& src) : s(src) {}
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) ++i;
    }
    bool lit(const char* t) {
        size_t n = std::strlen(t);
        if (s.compare(i, n, t) != 0) return false;
        i += n;
        return true;
    }
    bool value(Json& out, int depth) {
        if (depth > 64) { err = "nesting too deep"; return false; }
        ws();
        if (i >= s.size()) { err = "unexpected end"; return false; }
        char c = s[i];
        if (c == '{') {
            ++i;
            out.kind = Json::OBJ;
            ws();
            if (i < s.size() && s[i] == '}') { ++i; return true; }
            for (;;) {
                ws();
                Json key;
                if (i >= s.size() || s[i] != '"' || !string(key.str)) { if (err.empty()) err = "expected key"; return false; }
                ws();
                if (i >= s.size() || s[i] != ':') { err = "expected ':'"; return false; }
                ++i;
                Json v;
                if (!value(v, depth + 1)) return false;
                out.obj[key.str] = std::move(v);
                ws();
                if (i < s.size() && s[i] == ',') { ++i; continue; }
                if (i < s.size() && s[i] == '}') { ++i; return true; }
                err = "expected ',' or '}'";
                return false;
            }
        }
        if (c == '[') {
            ++i;
            out.kind = Json::ARR;
            ws();
            if (i < s.size() && s[i] == ']') { ++i; return true; }
            for (;;) {
                Json v;
                if (!value(v, depth + 1)) return false;
                out.arr.push_back(std::move(v));
                ws();
                if (i < s.size() && s[i] == ',') { ++i; continue; }
                if (i < s.size() && s[i] == ']') { ++i; return true; }
                err = "expected ',' or ']'";
                return false;
            }
        }
        if (c == '"') { out.kind = Json::STR; return string(out.str); }
        if (lit("true")) { out.kind = Json::BOOL; out.b = true; return true; }
        if (lit("false")) { out.kind = Json::BOOL; out.b = false; return true; }
        if (lit("null")) { out.kind = Json::NUL; return true; }
        size_t st = i;
        while (i < s.size() && (std::strchr("+-0123456789.eE", s[i]) != nullptr)) ++i;
        if (st == i) { err = "unexpected character"; return false; }
        char* end = nullptr;
        std::string tok = s.substr(st, i - st);
        out.num = std::strtod(tok.c_str(), &end);
        if (end == nullptr || *end != '\0') { err = "bad number"; return false; }
        out.kind = Json::NUM;
        return true;
    }
    bool string(std::string& out) {
        ++i;  // opening quote
        while (i < s.size() && s[i] != '"') {
            if (s[i] == '\\') {
                if (++i >= s.size()) break;
                char e = s[i];
                out.push_back(e == 'n' ? '\n' : e == 't' ? '\t' : e);
            } else {
                out.push_back(s[i]);
            }
            ++i;
        }
        if (i >= s.size()) { err = "unterminated string"; return false; }
        ++i;
        return true;
    }
};

int read_file(const std::string& path, std::string& out, const char* what) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) return fail(EE_ERR_IO, std::string("Could not open ") + what + ": " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    if (f.bad()) return fail(EE_ERR_IO, std::string("Failed to read ") + what + ": " + path);
    out = ss.str();
    return EE_OK;
}

int parse_json(const std::string& text, const std::string& path, Json& out) {
    JsonParser p(text);
    if (!p.value(out, 0)) return fail(EE_ERR_META, "Malformed meta JSON " + path + ": " + p.err);
    p.ws();
    if (p.i != text.size()) return fail(EE_ERR_META, "Malformed meta JSON " + path + ": trailing data");
    return EE_OK;
}

int json_int(const Json& o, const char* key, const std::string& path, int64_t& v) {
    const Json* j = o.get(key);
    if (j == nullptr) return fail(EE_ERR_META, std::string("Missing key: ") + key + " (" + path + ")");
    if (j->kind != Json::NUM) return fail(EE_ERR_META, std::string("Key is not a number: ") + key + " (" + path + ")");
    v = (int64_t)j->num;
    return EE_OK;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

struct Kernel {
    hipFunction_t fn = nullptr;
    int block = 0;
    int lds = 0;
    int kernarg = 0;                          // bytes of its by-value argument block (meta)
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

// Device address and size of ee_routed_linear_noalloc's workspace array on the
// current device (ee_noalloc.hip); returns a hipError_t value.
extern "C" int ee_noalloc_scratch_address(void** out, int64_t* bytes);

struct ee_engine {
    int device = -1;
    int cus = 0;                              // compute units: the persistent GEMM grids
    void* scratch = nullptr;                  // this device's copy of the no-alloc workspace
    int64_t scratch_bytes = 0;
    int scratch_rc = 0;                       // hipError_t of its lookup
    std::vector<hipModule_t> modules;
    std::unordered_map<std::string, Kernel> kernels;
    std::unordered_map<std::string, int64_t> options;
};

struct ee_module_engine {
    std::string func;
    int device = -1;
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
    int shared_mem = 0, num_warps = 0, block_m = 0, block_n = 0, static_lds = 0;
};

namespace {

int check_device(int device) {
    int cur = -1;
    EE_HIP(hipGetDevice(&cur), "hipGetDevice");
    if (cur != device)
        return fail(EE_ERR_INVALID_ARG, "engine was created on device " + std::to_string(device) +
                                            " but the current device is " + std::to_string(cur));
    return EE_OK;
}

const Kernel* find_kernel(const ee_engine* e, const std::string& name) {
    auto it = e->kernels.find(name);
    return it == e->kernels.end() ? nullptr : &it->second;
}

// Name of the last kernel this thread launched through launch() (ee_last_kernel).
thread_local std::string t_last_kernel;

template <typename Args>
int launch(ee_engine* e, const std::string& name, int64_t gx, int64_t gy, int block, Args args,
           ee_stream_t stream) {
    const Kernel* k = find_kernel(e, name);
    if (k == nullptr) return fail(EE_ERR_NOT_FOUND, "kernel not in the loaded code objects: " + name);
    if (gx <= 0 || gy <= 0) return EE_OK;
    if (gx > 0x7fffffff || gy > 65535) return fail(EE_ERR_UNSUPPORTED, "grid too large for " + name);
    if (block != k->block)
        return fail(EE_ERR_META, "launch block " + std::to_string(block) + " != meta block " +
                                     std::to_string(k->block) + " for " + name);
    if ((int)sizeof(Args) != k->kernarg)
        return fail(EE_ERR_INVALID_ARG, "argument block of " + name + " is " + std::to_string(sizeof(Args)) +
                                            " bytes but its code object takes " + std::to_string(k->kernarg));
    int rc = check_device(e->device);
    if (rc) return rc;
    void* params[] = {&args};
    EE_HIP(hipModuleLaunchKernel(k->fn, (unsigned)gx, (unsigned)gy, 1, (unsigned)block, 1, 1, 0,
                                 (hipStream_t)stream, params, nullptr),
           "hipModuleLaunchKernel(" + name + ")");
    t_last_kernel = name;
    return EE_OK;
}

// (VPT, WPR) for a register-resident row kernel: VPT 16-byte vectors per lane,
// WPR wave64s per row, VPT * WPR * 512 >= len: the fewest waves per row that
// still put min_waves waves on the chip (1024 SIMDs) with VPT <= max_vpt.  The
// softmax kernel takes 4096.  The quantisers take 4096 with VPT <= 6, measured
// from graph replays at the configs' and the Llama's shapes: [4096, 2048] 1 x 4
// 5.0 us (4 waves x 1: 6.1), [4096, 4096] 2 x 4 8.9 (4 x 2: 10.0), [4096, 5632]
// 2 x 6 12.4 (4 x 3: 12.8), [1024, 4096] 4 x 2 3.9 (2 x 4: 4.0).
bool pick_row_cfg(int64_t len, int64_t rows, int64_t forced_wpr, int& vpt, int& wpr, int64_t min_waves = 4096,
                  int max_vpt = 8) {
    const int options[3] = {1, 2, 4};
    int best = -1;
    for (int w : options) {
        if (forced_wpr && w != forced_wpr) continue;
        int v = (int)cdiv(len, 512LL * w);
        if (v < 1) v = 1;
        if (v > (forced_wpr ? 8 : max_vpt) && !(w == 4 && v <= 8)) continue;   // 4 waves: any VPT the kernels have
        best = w;
        if (forced_wpr || rows * w >= min_waves) break;
    }
    if (best < 0) return false;
    wpr = best;
    vpt = (int)cdiv(len, 512LL * best);
    if (vpt < 1) vpt = 1;
    return true;
}

// (VPT, WPR) for the softmax row kernel: WPR = 1..8 waves per row holding
// VPT <= 4 vectors per lane (the kernel keeps e in registers up to 4), with
// VPT * WPR * 512 >= len.  Among the layouts that cover the row: the one that
// fills the chip best (4096 waves of two or more vectors, else 2048 waves), then
// the least padding, then the fewest waves per row.  Rows longer than 4 * 8 * 512
// take eight waves and VPT 5..8.
bool pick_se_cfg(int64_t len, int64_t rows, int64_t forced_wpr, int& vpt, int& wpr) {
    int best_w = -1, best_v = 0;
    int64_t best_pad = 0;
    for (int w = 1; w <= 8; ++w) {
        if (forced_wpr && w != forced_wpr) continue;
        const int v = (int)std::max<int64_t>(1, cdiv(len, 512LL * w));
        if (v > 4 && !(w == 8 && v <= 8)) continue;
        const int64_t pad = (int64_t)v * w * 512 - len;
        // 2048 waves (8 per CU) keep HBM busy; 4096 waves of two or more vectors also
        // halve each wave's share of the row's exponentials, which at [1024, 4096]
        // (2048 waves of 4 vectors otherwise) is the longest phase of a wave's life:
        // 4 waves x 2 vectors 6.01 us cold against 2 x 4 6.20 us.  At [4096, 4096]
        // 2 x 4 already gives 8192 waves (13.45 us against 4 x 2's 14.44 us).
        auto fill = [&](int ww, int vv) { return rows * ww >= 4096 && vv >= 2 ? 2 : rows * ww >= 2048 ? 1 : 0; };
        if (best_w < 0) { best_w = w; best_v = v; best_pad = pad; continue; }
        const int f = fill(w, v), best_f = fill(best_w, best_v);
        // prefer filling the chip, then least padding, then fewer waves per row
        if (f > best_f || (f == best_f && pad < best_pad)) {
            best_w = w; best_v = v; best_pad = pad;
        }
    }
    if (best_w < 0) return false;
    // A power-of-two wave count (1, 2, 4, 8: the block's waves spread evenly over the
    // 4 SIMDs) over a non-power-of-two one when it fills the chip too and at least
    // 7/8 of its row capacity is used: [4096, 14336] takes 8 waves x 4 vectors
    // (12.5% padding) over 7 x 4 (none), 42.6 vs 44.1 us cold.
    if (!forced_wpr && (best_w & (best_w - 1)) != 0) {
        const bool best_fills = rows * best_w >= 2048;
        for (int w = 1; w <= 8; w *= 2) {
            const int v = (int)std::max<int64_t>(1, cdiv(len, 512LL * w));
            if (v > 4 && !(w == 8 && v <= 8)) continue;
            const int64_t cap = (int64_t)v * w * 512;
            if ((rows * w >= 2048 || !best_fills) && len * 8 >= cap * 7) {
                best_w = w;
                best_v = v;
                break;
            }
        }
    }
    wpr = best_w;
    vpt = best_v;
    return true;
}

int64_t opt(const ee_engine* e, const char* key) {
    auto it = e->options.find(key);
    return it == e->options.end() ? 0 : it->second;
}

// Workgroups of a persistent GEMM over `tiles` tiles, or 0 for the one-tile-per-
// workgroup kernels.  Auto: one workgroup per CU (a multiple of 8, so each XCD
// gets the same share) once there are more tiles than CUs.  Option
// "gemm_persist": 1 = never, n >= 2 = always, with min(n, tiles) workgroups.
int64_t persist_grid(const ee_engine* e, int64_t tiles) {
    const int64_t v = opt(e, "gemm_persist");
    if (v == 1) return 0;
    if (v >= 2) return std::min(v, tiles);
    const int64_t g = e->cus >= 8 ? (e->cus & ~7) : e->cus;
    return tiles > e->cus ? g : 0;
}

}  // namespace

// ============================================================================ API

EE_EXPORT const char* ee_last_error(void) { return g_err.c_str(); }
EE_EXPORT int ee_abi_version(void) { return EE_ABI_VERSION; }

EE_EXPORT int ee_engine_create(const char* lib_dir, ee_engine** out) {
    if (out == nullptr) return fail(EE_ERR_INVALID_ARG, "out must not be NULL");
    *out = nullptr;
    if (lib_dir == nullptr) return fail(EE_ERR_INVALID_ARG, "lib_dir must not be NULL");
    const std::string dir(lib_dir);
    const std::string meta_path = dir + "/entropy_engine_meta.json";
    std::string text;
    int rc = read_file(meta_path, text, "meta JSON");
    if (rc) return rc;
    Json meta;
    if ((rc = parse_json(text, meta_path, meta))) return rc;
    const Json* fmt = meta.get("format");
    if (fmt == nullptr || fmt->kind != Json::STR || fmt->str != "entropy-engine-meta/1")
        return fail(EE_ERR_META, "Missing key: format (expected entropy-engine-meta/1) in " + meta_path);
    const Json* cos = meta.get("code_objects");
    const Json* kns = meta.get("kernels");
    if (cos == nullptr || cos->kind != Json::OBJ) return fail(EE_ERR_META, "Missing key: code_objects (" + meta_path + ")");
    if (kns == nullptr || kns->kind != Json::OBJ) return fail(EE_ERR_META, "Missing key: kernels (" + meta_path + ")");

    // Validate the whole meta, then read every code object, before touching HIP.
    struct KSpec { std::string co; int64_t block, lds, kernarg; };
    std::map<std::string, KSpec> specs;
    for (const auto& kv : kns->obj) {
        const Json* co = kv.second.get("code_object");
        if (co == nullptr || co->kind != Json::STR)
            return fail(EE_ERR_META, "Missing key: code_object for kernel " + kv.first + " (" + meta_path + ")");
        if (cos->get(co->str) == nullptr)
            return fail(EE_ERR_META, "kernel " + kv.first + " names unknown code object " + co->str);
        KSpec s{co->str, 0, 0, 0};
        if ((rc = json_int(kv.second, "block", meta_path, s.block))) return rc;
        if ((rc = json_int(kv.second, "lds", meta_path, s.lds))) return rc;
        if ((rc = json_int(kv.second, "kernarg", meta_path, s.kernarg))) return rc;
        if (s.block <= 0 || s.block > 1024) return fail(EE_ERR_META, "bad block size for " + kv.first);
        if (s.kernarg <= 0 || s.kernarg > 4096) return fail(EE_ERR_META, "bad kernarg size for " + kv.first);
        specs[kv.first] = s;
    }

    struct Pending { std::string file, bytes; };
    std::map<std::string, Pending> blobs;
    for (const auto& kv : cos->obj) {
        const Json* file = kv.second.get("file");
        if (file == nullptr || file->kind != Json::STR)
            return fail(EE_ERR_META, "Missing key: file for code object " + kv.first + " (" + meta_path + ")");
        Pending p;
        p.file = dir + "/" + file->str;
        if ((rc = read_file(p.file, p.bytes, "code object"))) return rc;
        if (p.bytes.size() < 4 || std::memcmp(p.bytes.data(), "\x7f" "ELF", 4) != 0)
            return fail(EE_ERR_IO, "Not an ELF code object: " + p.file);
        blobs[kv.first] = std::move(p);
    }
    std::unique_ptr<ee_engine> e(new ee_engine());
    auto cleanup = [&]() {
        for (hipModule_t m : e->modules) (void)hipModuleUnload(m);
        e->modules.clear();
    };
    if (hipGetDevice(&e->device) != hipSuccess) return fail(EE_ERR_HIP, "hipGetDevice failed (no GPU?)");
    if (hipDeviceGetAttribute(&e->cus, hipDeviceAttributeMultiprocessorCount, e->device) != hipSuccess ||
        e->cus <= 0)
        return fail(EE_ERR_HIP, "hipDeviceGetAttribute(MultiprocessorCount) failed");
    std::map<std::string, hipModule_t> loaded;
    for (auto& kv : blobs) {
        hipModule_t m = nullptr;
        hipError_t err = hipModuleLoadData(&m, kv.second.bytes.data());
        if (err != hipSuccess) {
            cleanup();
            return fail(EE_ERR_HIP, "hipModuleLoadData failed for " + kv.second.file + ": " + hipGetErrorString(err));
        }
        e->modules.push_back(m);
        loaded[kv.first] = m;
    }
    for (auto& kv : specs) {
        Kernel k;
        hipError_t err = hipModuleGetFunction(&k.fn, loaded[kv.second.co], kv.first.c_str());
        if (err != hipSuccess) {
            cleanup();
            return fail(EE_ERR_NOT_FOUND, "hipModuleGetFunction failed for '" + kv.first + "' in " +
                                              blobs[kv.second.co].file + ": " + hipGetErrorString(err));
        }
        int max_threads = 0, lds = 0;
        if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, k.fn) != hipSuccess ||
            hipFuncGetAttribute(&lds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, k.fn) != hipSuccess) {
            cleanup();
            return fail(EE_ERR_HIP, "hipFuncGetAttribute failed for " + kv.first);
        }
        if (max_threads < kv.second.block || lds != kv.second.lds) {
            cleanup();
            return fail(EE_ERR_META, "meta of " + kv.first + " (block " + std::to_string(kv.second.block) +
                                         ", lds " + std::to_string(kv.second.lds) + ") disagrees with the code object (max threads " +
                                         std::to_string(max_threads) + ", lds " + std::to_string(lds) + ")");
        }
        k.block = (int)kv.second.block;
        k.lds = lds;
        k.kernarg = (int)kv.second.kernarg;
        e->kernels[kv.first] = k;
    }
    // This device's copy of ee_routed_linear_noalloc's workspace; a failed lookup
    // only disables that entry point (it reports the HIP error).
    e->scratch_rc = ee_noalloc_scratch_address(&e->scratch, &e->scratch_bytes);
    *out = e.release();
    return EE_OK;
}

EE_EXPORT int ee_engine_destroy(ee_engine* eng) {
    if (eng == nullptr) return EE_OK;
    int rc = EE_OK;
    for (hipModule_t m : eng->modules)
        if (hipModuleUnload(m) != hipSuccess) rc = fail(EE_ERR_HIP, "hipModuleUnload failed");
    delete eng;
    return rc;
}

EE_EXPORT int ee_engine_set_option(ee_engine* eng, const char* key, int64_t value) {
    if (eng == nullptr || key == nullptr) return fail(EE_ERR_INVALID_ARG, "engine and key must not be NULL");
    const std::string k(key);
    if (k == "se_wpr") {
        if (value < 0 || value > 8) return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto) or 1..8");
    } else if (k == "se_nt") {
        if (value < 0 || value > 2) return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 1 (off) or 2 (on)");
    } else if (k == "se_rpw") {
        if (value != 0 && value != 1 && value != 2 && value != 4)
            return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 1, 2 or 4");
    } else if (k == "quant_wpr") {
        if (value != 0 && value != 1 && value != 2 && value != 4)
            return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 1, 2 or 4");
    } else if (k == "gemm_variant") {
        if (value < 0 || value > 2) return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 1 or 2");
    } else if (k == "routed_unfused") {
        if (value != 0 && value != 1) return fail(EE_ERR_INVALID_ARG, k + " must be 0 or 1");
    } else if (k == "gemm_persist") {
        if (value < 0 || value > 65535) return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 1 (off) or a grid >= 2");
    } else if (k == "gemm_tile") {
        if (value != 0 && value != 128 && value != 256)
            return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 128 or 256");
    } else if (k == "gemm_tile_n") {
        if (value != 0 && value != 128 && value != 256)
            return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 128 or 256");
    } else if (k == "gemm_waves") {
        if (value != 0 && value != 4 && value != 8)
            return fail(EE_ERR_INVALID_ARG, k + " must be 0 (auto), 4 or 8");
    } else {
        return fail(EE_ERR_INVALID_ARG, "unknown option: " + k);
    }
    eng->options[k] = value;
    return EE_OK;
}

EE_EXPORT int ee_engine_device(const ee_engine* eng) { return eng ? eng->device : -1; }

EE_EXPORT const char* ee_last_kernel(void) { return t_last_kernel.c_str(); }

EE_EXPORT int ee_softmax_entropy(ee_engine* eng, const void* x, void* p, float* h, int64_t rows, int32_t S,
                                 int64_t ld_x, int64_t ld_p, int32_t causal, int32_t* tier, double tau_low,
                                 double tau_high, ee_stream_t stream) {
    if (eng == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (x == nullptr || h == nullptr) return fail(EE_ERR_INVALID_ARG, "x and h must not be NULL");
    if (rows < 0 || S <= 0) return fail(EE_ERR_INVALID_ARG, "need rows >= 0 and S > 0");
    if (ld_x < S || (p != nullptr && ld_p < S)) return fail(EE_ERR_INVALID_ARG, "row stride smaller than S");
    if (causal != 0 && causal != 1) return fail(EE_ERR_INVALID_ARG, "causal must be 0 or 1");
    if (!aligned(x, 2) || !aligned(p, 2) || !aligned(h, 4) || !aligned(tier, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (rows == 0) return EE_OK;
    EeSoftmaxArgs a{(const uint16_t*)x, (uint16_t*)p, h, tier, rows, ld_x, ld_p, S, causal, tau_low, tau_high};
    // Non-temporal loads of the logits (the _nt kernels of the multi-wave layouts; option
    // "se_nt": 0 auto, 1 off, 2 on).  Measured on MI355X at [4096, 14336]: logits read
    // from HBM (rotating buffers) 3-5% faster; logits just written by a producer kernel
    // (the pipeline's case) 2% slower; the same buffer again 11% slower.  Automatic takes
    // them only where the logits and probabilities together exceed the 256 MiB Infinity
    // Cache, so that logits cannot have stayed there ([8192, 8192]: a tie after a producer).
    const int64_t nt_opt = opt(eng, "se_nt");
    const int64_t se_bytes = rows * S * 2 * (p != nullptr ? 2 : 1);
    const bool nt = nt_opt == 2 || (nt_opt == 0 && se_bytes > (int64_t(256) << 20));
    const bool vec_ok = aligned(x, 16) && aligned(p, 16) && ld_x % 8 == 0 && (p == nullptr || ld_p % 8 == 0);
    int vpt = 0, wpr = 0;
    if (vec_ok && pick_se_cfg(S, rows, opt(eng, "se_wpr"), vpt, wpr)) {
        // Short single-wave rows: several rows per wave (their loads issued together)
        // once there are rows enough to keep every CU busy.  Option "se_rpw": 1 = one
        // row per wave, 2 or 4 = that many where the variant exists.
        if (wpr == 1 && vpt <= 2) {
            const int64_t f = opt(eng, "se_rpw");
            // measured at [131072, 512]: 2 rows per wave -8% (causal) to -11%; 4 no better than 2
            const int rpw = f ? (int)f : (rows >= 32768 ? 2 : 1);
            const std::string rname = "eek_softmax_entropy_v" + std::to_string(vpt) + "_r" + std::to_string(rpw);
            if (rpw > 1 && find_kernel(eng, rname))
                return launch(eng, rname, cdiv(rows, 4LL * rpw), 1, EE_BLOCK, a, stream);
        }
        std::string name = "eek_softmax_entropy_v" + std::to_string(vpt) + "_w" + std::to_string(wpr);
        if (nt && find_kernel(eng, name + "_nt")) name += "_nt";
        const int rpb = wpr == 1 ? 4 : (wpr == 2 ? 2 : 1);      // rows per block (kernel's SeGeom)
        const Kernel* k = find_kernel(eng, name);
        return launch(eng, name, cdiv(rows, rpb), 1, k ? k->block : rpb * wpr * 64, a, stream);
    }
    return launch(eng, "eek_softmax_entropy_generic", cdiv(rows, 4), 1, EE_BLOCK, a, stream);
}

// The register-resident row kernel when rows are 16-byte aligned and fit, else the generic one.
static int launch_quant(ee_engine* eng, const EeQuantArgs& a, ee_stream_t stream) {
    const bool vec_ok = aligned(a.x, 16) && aligned(a.codes, 8) && a.ld_x % 8 == 0 && a.ld_c % 8 == 0;
    int vpt = 0, wpr = 0;
    if (vec_ok && pick_row_cfg(a.K, a.M, opt(eng, "quant_wpr"), vpt, wpr, 4096, 6)) {
        const std::string name = "eek_quant_v" + std::to_string(vpt) + "_w" + std::to_string(wpr);
        return launch(eng, name, cdiv(a.M, 4 / wpr), 1, EE_BLOCK, a, stream);
    }
    return launch(eng, "eek_quant_generic", cdiv(a.M, 4), 1, EE_BLOCK, a, stream);
}

EE_EXPORT int ee_quant_act(ee_engine* eng, const void* x, int64_t M, int64_t K, int64_t ld_x, int32_t mode,
                           void* codes, int64_t ld_c, float* scale, const int32_t* idx, const int32_t* counts,
                           int32_t tier, ee_stream_t stream) {
    if (eng == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (x == nullptr || codes == nullptr || scale == nullptr)
        return fail(EE_ERR_INVALID_ARG, "x, codes and scale must not be NULL");
    if (M < 0 || K <= 0) return fail(EE_ERR_INVALID_ARG, "need M >= 0 and K > 0");
    if (ld_x < K || ld_c < K) return fail(EE_ERR_INVALID_ARG, "row stride smaller than K");
    if (mode == EE_QUANT_F8_TENSOR)
        return fail(EE_ERR_INVALID_ARG, "EE_QUANT_F8_TENSOR needs a workspace: use ee_quant_tensor_f8");
    if (mode < EE_QUANT_I8_DISPATCH || mode > EE_QUANT_F8_ROW) return fail(EE_ERR_INVALID_ARG, "unknown quant mode");
    if ((idx != nullptr) && counts == nullptr) return fail(EE_ERR_INVALID_ARG, "idx needs counts");
    if (counts != nullptr && (tier < 0 || tier > 2)) return fail(EE_ERR_INVALID_ARG, "tier must be 0, 1 or 2");
    if (!aligned(x, 2) || !aligned(scale, 4) || !aligned(idx, 4) || !aligned(counts, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (M == 0) return EE_OK;
    EeQuantArgs a{(const uint16_t*)x, codes, scale, idx, counts, M, K, ld_x, ld_c, mode, counts ? tier : 0,
                  nullptr, 0};
    return launch_quant(eng, a, stream);
}

EE_EXPORT int ee_quant_tensor_f8(ee_engine* eng, const void* x, int64_t M, int64_t K, int64_t ld_x, uint8_t* codes,
                                 int64_t ld_c, float* scale, float* ws, ee_stream_t stream) {
    if (eng == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (x == nullptr || codes == nullptr || scale == nullptr || ws == nullptr)
        return fail(EE_ERR_INVALID_ARG, "x, codes, scale and ws must not be NULL");
    if (M < 0 || K <= 0) return fail(EE_ERR_INVALID_ARG, "need M >= 0 and K > 0");
    if (ld_x < K || ld_c < K) return fail(EE_ERR_INVALID_ARG, "row stride smaller than K");
    if (!aligned(x, 2) || !aligned(scale, 4) || !aligned(ws, 4)) return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (M == 0) return EE_OK;
    const int64_t nblk = std::min<int64_t>(EE_TENSOR_WS_FLOATS, cdiv(M, 4));
    EeAbsmaxArgs p{(const uint16_t*)x, (uint32_t*)ws, M, K, ld_x};
    int rc = launch(eng, "eek_absmax_partial", nblk, 1, EE_BLOCK, p, stream);
    if (rc) return rc;
    EeQuantArgs a{(const uint16_t*)x, codes, scale, nullptr, nullptr, M, K, ld_x, ld_c, EE_QUANT_F8_TENSOR, 0,
                  (const uint32_t*)ws, (int32_t)nblk};
    return launch_quant(eng, a, stream);
}

EE_EXPORT int ee_quant_weight_i8(ee_engine* eng, const void* w, int64_t N, int64_t K, int64_t ld_w,
                                 int8_t* codes_nk, int64_t ld_c, float* scale, ee_stream_t stream) {
    // Per output channel n: the f32-scale, round-half-even, clamp(+-127) quantiser.
    return ee_quant_act(eng, w, N, K, ld_w, EE_QUANT_I8_ENGINE, codes_nk, ld_c, scale, nullptr, nullptr, 0, stream);
}

EE_EXPORT int ee_transpose_i8(ee_engine* eng, const int8_t* src, int64_t R, int64_t C, int64_t ld_src,
                              int8_t* dst, int64_t ld_dst, ee_stream_t stream) {
    if (eng == nullptr || src == nullptr || dst == nullptr) return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (R < 0 || C < 0 || ld_src < C || ld_dst < R) return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (cdiv(R, 64) > 65535) return fail(EE_ERR_UNSUPPORTED, "too many rows for ee_transpose_i8");
    EeWeightArgs a{src, dst, nullptr, nullptr, R, C, ld_src, ld_dst};
    return launch(eng, "eek_transpose_i8", cdiv(C, 64), cdiv(R, 64), EE_BLOCK, a, stream);
}

EE_EXPORT int ee_pack_b_f8(ee_engine* eng, const int8_t* codes_nk, int64_t N, int64_t K, int64_t ld_src,
                           uint8_t* dst, int64_t ld_dst, ee_stream_t stream) {
    if (eng == nullptr || codes_nk == nullptr || dst == nullptr) return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (N < 0 || K < 0 || ld_src < K || ld_dst < K) return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    EeWeightArgs a{codes_nk, dst, nullptr, nullptr, N, K, ld_src, ld_dst};
    int64_t g = cdiv(N * K, EE_BLOCK);
    return launch(eng, "eek_pack_b_f8", g > 16384 ? 16384 : g, 1, EE_BLOCK, a, stream);
}

EE_EXPORT int ee_pack_b_f16(ee_engine* eng, const int8_t* codes_nk, const float* scale, int64_t N, int64_t K,
                            int64_t ld_src, void* dst, int64_t ld_dst, ee_stream_t stream) {
    if (eng == nullptr || codes_nk == nullptr || scale == nullptr || dst == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (N < 0 || K < 0 || ld_src < K || ld_dst < K) return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (!aligned(dst, 2) || !aligned(scale, 4)) return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    EeWeightArgs a{codes_nk, dst, nullptr, scale, N, K, ld_src, ld_dst};
    int64_t g = cdiv(N * K, EE_BLOCK);
    return launch(eng, "eek_pack_b_f16", g > 16384 ? 16384 : g, 1, EE_BLOCK, a, stream);
}

// sw = 1: SwiGLU epilogue (b_nk gate|up interleaved in blocks of 32 rows; c is act [M, N/2]).
static int gemm_impl(ee_engine* eng, int32_t kind, const void* a, int64_t lda, const void* b_nk, int64_t ldb,
                     void* c, int64_t ldc, const float* a_scale, const float* b_scale, int32_t M, int32_t N,
                     int32_t K, const int32_t* a_idx, const int32_t* c_idx, const int32_t* counts, int32_t tier,
                     int32_t* acc_out, int sw, ee_stream_t stream) {
    if (eng == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (kind < EE_GEMM_I8 || kind > EE_GEMM_W8A16) return fail(EE_ERR_INVALID_ARG, "unknown GEMM kind");
    if (a == nullptr || b_nk == nullptr || c == nullptr) return fail(EE_ERR_INVALID_ARG, "a, b and c must not be NULL");
    if (kind != EE_GEMM_F16 && kind != EE_GEMM_W8A16 && (a_scale == nullptr || b_scale == nullptr))
        return fail(EE_ERR_INVALID_ARG, "a_scale and b_scale are required for the INT8 and FP8 tiers");
    if (kind == EE_GEMM_W8A16) {
        // fp16 A, int8 B codes + f32 scales, dequantised in the kernel: one pipeline (K % 64 == 0)
        if (b_scale == nullptr) return fail(EE_ERR_INVALID_ARG, "b_scale is required for W8A16");
        if (acc_out != nullptr) return fail(EE_ERR_INVALID_ARG, "acc_out is INT8 only");
        if (M < 0 || N <= 0 || K <= 0) return fail(EE_ERR_INVALID_ARG, "need M >= 0, N > 0, K > 0");
        if (lda < K || ldb < K || ldc < (sw ? N / 2 : N))
            return fail(EE_ERR_INVALID_ARG, "leading dimension smaller than the row");
        if (K % 64 != 0 || lda % 8 != 0 || ldb % 16 != 0 || N % 4 != 0 || ldc % 4 != 0)
            return fail(EE_ERR_UNSUPPORTED, "W8A16 needs K % 64 == 0, lda % 8 == 0, ldb % 16 == 0, N % 4 == 0, "
                                            "ldc % 4 == 0");
        if (sw && (N % 64 != 0 || ldc % 8 != 0 || !aligned(c, 16)))
            return fail(EE_ERR_UNSUPPORTED, "SwiGLU GEMM needs N % 64 == 0, ld_act % 8 == 0, a 16-byte aligned act");
        if (!aligned(a, 16) || !aligned(b_nk, 16) || !aligned(c, 8) || !aligned(b_scale, 4) || !aligned(a_idx, 4) ||
            !aligned(c_idx, 4) || !aligned(counts, 4))
            return fail(EE_ERR_INVALID_ARG, "misaligned pointer (a, b: 16 B; c: 8 B; b_scale, indices: 4 B)");
        if ((a_idx != nullptr || c_idx != nullptr) && counts == nullptr)
            return fail(EE_ERR_INVALID_ARG, "a_idx / c_idx need counts");
        if (counts != nullptr && (tier < 0 || tier > 2)) return fail(EE_ERR_INVALID_ARG, "tier must be 0, 1 or 2");
        if (M == 0) return EE_OK;
        EeGemmArgs g{a, b_nk, (uint16_t*)c, nullptr, nullptr, b_scale, a_idx, c_idx, counts, lda, ldb, ldc,
                     M, N, K, counts ? tier : 0, sw};
        // The four-wave 256-row tiles (eek_gemm4w[n128]_w8a16) wherever EE_GEMM_F16 on
        // eek_pack_b_f16's weights would run eek_gemm4w[n128]_f16 (the conditions
        // below): the same MFMAs on the same weight values in the same K order, so
        // the same bits, with B streamed at 1 byte per element.
        {
            const int64_t tiles = cdiv(M, 128) * cdiv(N, 128);
            const bool off32 = 255 * std::max(lda * 2, ldb) + K * 2 < (int64_t(1) << 32);
            const int64_t tile_opt = opt(eng, "gemm_tile"), tn_opt = opt(eng, "gemm_tile_n");
            if (counts == nullptr && K >= 128 && tile_opt != 128 && off32 && opt(eng, "gemm_variant") != 2 &&
                opt(eng, "gemm_waves") != 8 && (tile_opt == 256 || tiles > eng->cus)) {
                const int64_t gcu = eng->cus >= 8 ? (eng->cus & ~7) : eng->cus;
                const int64_t t256 = cdiv(M, 256) * cdiv(N, 256), t128 = cdiv(M, 256) * cdiv(N, 128);
                const bool narrow = tn_opt == 128 || (tn_opt == 0 && 2 * t256 <= gcu);
                const std::string n4 = std::string(narrow ? "eek_gemm4wn128_w8a16" : "eek_gemm4w_w8a16") +
                                       (sw ? "_swiglu" : "");
                const Kernel* k4 = find_kernel(eng, n4);
                if (k4 != nullptr) {
                    const int64_t tt = narrow ? t128 : t256;
                    int64_t g4 = persist_grid(eng, tt);
                    if (g4 <= 0) g4 = std::min<int64_t>(tt, gcu);
                    if (g4 <= 0) g4 = tt;
                    return launch(eng, n4, g4, 1, k4->block, g, stream);
                }
            }
        }
        const std::string name = sw ? "eek_gemm_w8a16_swiglu" : "eek_gemm_w8a16";
        const Kernel* k = find_kernel(eng, name);
        return launch(eng, name, cdiv(M, 128) * cdiv(N, 128), 1, k ? k->block : EE_BLOCK, g, stream);
    }
    if (acc_out != nullptr && kind != EE_GEMM_I8) return fail(EE_ERR_INVALID_ARG, "acc_out is INT8 only");
    if (M < 0 || N <= 0 || K <= 0) return fail(EE_ERR_INVALID_ARG, "need M >= 0, N > 0, K > 0");
    const int64_t esz = (kind == EE_GEMM_F16) ? 2 : 1;
    if (lda < K || ldb < K || ldc < (sw ? N / 2 : N))
        return fail(EE_ERR_INVALID_ARG, "leading dimension smaller than the row");
    if (sw && (N % 64 != 0 || ldc % 8 != 0 || !aligned(c, 16) || (K * esz) % 128 != 0 || acc_out != nullptr))
        return fail(EE_ERR_UNSUPPORTED, "SwiGLU GEMM needs N % 64 == 0 (gate|up interleaved in blocks of 32), "
                                        "ld_act % 8 == 0, a 16-byte aligned act, K * element size % 128 == 0 "
                                        "and no acc_out");
    if ((K * esz) % 16 != 0) return fail(EE_ERR_UNSUPPORTED, "K * element size must be a multiple of 16 bytes");
    if ((lda * esz) % 16 != 0 || (ldb * esz) % 16 != 0)
        return fail(EE_ERR_UNSUPPORTED, "lda and ldb must be multiples of 16 bytes");
    if (N % 4 != 0 || ldc % 4 != 0) return fail(EE_ERR_UNSUPPORTED, "N and ldc must be multiples of 4");
    if (!aligned(a, 16) || !aligned(b_nk, 16) || !aligned(c, 8) || !aligned(acc_out, 16) ||
        !aligned(a_scale, 4) || !aligned(b_scale, 16) || !aligned(a_idx, 4) || !aligned(c_idx, 4) ||
        !aligned(counts, 4))
        return fail(EE_ERR_INVALID_ARG,
                    "misaligned pointer (a, b, b_scale, acc: 16 B; c: 8 B; a_scale, indices: 4 B)");
    if ((a_idx != nullptr || c_idx != nullptr) && counts == nullptr)
        return fail(EE_ERR_INVALID_ARG, "a_idx / c_idx need counts");
    if (counts != nullptr && (tier < 0 || tier > 2)) return fail(EE_ERR_INVALID_ARG, "tier must be 0, 1 or 2");
    if (M == 0) return EE_OK;
    EeGemmArgs g{a, b_nk, (uint16_t*)c, acc_out, a_scale, b_scale, a_idx, c_idx, counts, lda, ldb, ldc,
                 M, N, K, counts ? tier : 0, sw};
    // The pipelined kernels stream whole 128-byte K stages; other K take the fallback.
    // Two pipelines: loader waves + MFMA waves (eek_gemm_*), and eight waves that
    // each load and compute (eek_gemm_*_w8).  Measured on MI355X (identical data,
    // interleaved runs), both on 16x16x64 MFMAs for INT8: the loader-wave form is
    // 3-4.5% faster for INT8 grids of at most one tile per CU (1024 x 4096 x 4096:
    // 18.8 against 19.4 us; 821 and 256 rows alike) and level at 2048^3; with
    // several tiles per CU it was ~5% faster already.  FP8 keeps the loader-wave
    // form (its 8-wave form spills).  The FP16 tier takes the loader-wave form
    // unless gemm_variant = 2: its 8-wave form splits K between wave pairs, an f32
    // order no other kernel (the 256 tiles, the routed grids) shares, and every
    // FP16 row must get the same bits whatever the shape or routing.
    static const char* names[3] = {"eek_gemm_i8", "eek_gemm_f8", "eek_gemm_f16"};
    const int64_t tiles = cdiv(M, 128) * cdiv(N, 128);
    std::string name = std::string(names[kind]) + (((K * esz) % 128 == 0) ? "" : "_generic");
    int64_t grid = tiles;
    // 256 x 256 tiles (eek_gemm256_*) where the 128-tile grid would take more
    // than one round of the CUs: they stream half the operand bytes per MFMA op.
    // They sum K in the loader-wave kernels' order, so every tier gives the same
    // bits either way (the FP16 tier's 8-wave split-K pipeline, gemm_variant 2,
    // has its own order and keeps the 128 tiles).
    const int64_t tile_opt = opt(eng, "gemm_tile");
    const int64_t variant = opt(eng, "gemm_variant");
    // (The kernels address a 256-row panel with 32-bit byte offsets.)
    const bool off32 = 255 * std::max(lda, ldb) * esz + K * esz < (int64_t(1) << 32);
    if ((K * esz) % 128 == 0 && counts == nullptr && tile_opt != 128 && off32 &&
        !(kind == EE_GEMM_F16 && variant == 2) && (tile_opt == 256 || tiles > eng->cus)) {
        static const char* names256[3] = {"eek_gemm256_i8", "eek_gemm256_f8", "eek_gemm256_f16"};
        static const char* names128[3] = {"eek_gemm256n128_i8", "eek_gemm256n128_f8", "eek_gemm256n128_f16"};
        // Tile width: 256 x 128 where the 256 x 256 grid would keep at most half the CUs
        // busy.  Measured (eager, same box): 4096 x 2048 x 2048 INT8 22.5 against 27.6 us,
        // 4096 x 5632 x 2048 51.5 against 61.1 (FP8 -17%); but at N = 2560 (160 tiles of
        // 256 x 256) 37.6 against 28.1, and a 256 x 256 grid whose last round is half
        // full (4096 x 14336: 3.5 rounds) is still faster than 7 rounds of 256 x 128
        // tiles (229 against 253 us): those stream 1.5x the bytes per MFMA op.
        // Option "gemm_tile_n": 0 auto, 128 or 256 forced.
        const int64_t tn_opt = opt(eng, "gemm_tile_n");
        const int64_t gcu = eng->cus >= 8 ? (eng->cus & ~7) : eng->cus;
        const int64_t t256 = cdiv(M, 256) * cdiv(N, 256), t128 = cdiv(M, 256) * cdiv(N, 128);
        const bool narrow = tn_opt == 128 || (tn_opt == 0 && 2 * t256 <= gcu);
        std::string n256 = std::string(narrow ? names128[kind] : names256[kind]) + (sw ? "_swiglu" : "");
        // Four waves per workgroup, each a 128 x (tile width / 2) quarter of the tile
        // (eek_gemm4w*: the same tiles, deal and K order, so the same bits), where a
        // tile has at least two K stages.  Measured on MI355X (same inputs, alternating
        // launches), 8 against 4 waves: 4096^3 INT8 55.7 / 54.0 us, FP8 54.2 / 54.0,
        // FP16 106.8 / 99.5; 4096 x 4096 x 14336 INT8 196 / 185, FP8 187 / 186, FP16
        // 379 / 349.  Option "gemm_waves": 0 auto (4), 4 or 8.
        static const char* names4w[3] = {"eek_gemm4w_i8", "eek_gemm4w_f8", "eek_gemm4w_f16"};
        static const char* names4w128[3] = {"eek_gemm4wn128_i8", "eek_gemm4wn128_f8", "eek_gemm4wn128_f16"};
        const int64_t waves_opt = opt(eng, "gemm_waves");
        if (waves_opt != 8 && K * esz >= 256) {
            const std::string n4 = std::string(narrow ? names4w128[kind] : names4w[kind]) + (sw ? "_swiglu" : "");
            if (find_kernel(eng, n4) != nullptr) n256 = n4;
        }
        const Kernel* k256 = find_kernel(eng, n256);
        if (k256 != nullptr) {
            const int64_t tt = narrow ? t128 : t256;
            int64_t g256 = persist_grid(eng, tt);
            if (g256 <= 0) g256 = std::min<int64_t>(tt, gcu);
            if (g256 <= 0) g256 = tt;
            return launch(eng, n256, g256, 1, k256->block, g, stream);
        }
    }
    if ((K * esz) % 128 == 0) {
        const int64_t v = variant;
        const bool w8 = v == 2;
        if (w8 && find_kernel(eng, name + "_w8")) {
            name += "_w8";
        } else if (kind != EE_GEMM_F16 && counts == nullptr) {
            // several tiles per CU: the persistent loader-wave kernel (same K order, same bits)
            const int64_t pg = persist_grid(eng, tiles);
            if (pg > 0 && find_kernel(eng, name + "_persist")) {
                name += "_persist";
                grid = pg;
            }
        }
    }
    if (sw) name += "_swiglu";
    const Kernel* k = find_kernel(eng, name);
    return launch(eng, name, grid, 1, k ? k->block : EE_BLOCK, g, stream);
}

EE_EXPORT int ee_gemm(ee_engine* eng, int32_t kind, const void* a, int64_t lda, const void* b_nk, int64_t ldb,
                      void* c, int64_t ldc, const float* a_scale, const float* b_scale, int32_t M, int32_t N,
                      int32_t K, const int32_t* a_idx, const int32_t* c_idx, const int32_t* counts, int32_t tier,
                      int32_t* acc_out, ee_stream_t stream) {
    return gemm_impl(eng, kind, a, lda, b_nk, ldb, c, ldc, a_scale, b_scale, M, N, K, a_idx, c_idx, counts, tier,
                     acc_out, 0, stream);
}

EE_EXPORT int ee_gemm_swiglu(ee_engine* eng, int32_t kind, const void* a, int64_t lda, const void* b_nk,
                             int64_t ldb, void* act, int64_t ld_act, const float* a_scale, const float* b_scale,
                             int32_t M, int32_t N, int32_t K, const int32_t* a_idx, const int32_t* c_idx,
                             const int32_t* counts, int32_t tier, ee_stream_t stream) {
    return gemm_impl(eng, kind, a, lda, b_nk, ldb, act, ld_act, a_scale, b_scale, M, N, K, a_idx, c_idx, counts,
                     tier, nullptr, 1, stream);
}

EE_EXPORT int ee_route(ee_engine* eng, const float* h, int64_t rows, double tau_low, double tau_high,
                       int32_t* tier, int32_t* idx, int32_t* counts, ee_stream_t stream) {
    if (eng == nullptr || h == nullptr || tier == nullptr || idx == nullptr || counts == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (rows < 0 || rows > 0x7fffffff) return fail(EE_ERR_INVALID_ARG, "rows out of range");
    if (!aligned(h, 4) || !aligned(tier, 4) || !aligned(idx, 4) || !aligned(counts, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    EeRouteArgs a{h, tier, idx, counts, rows, tau_low, tau_high, 1, 1};
    return launch(eng, "eek_route", 1, 1, 1024, a, stream);
}

EE_EXPORT int ee_route_heads(ee_engine* eng, const float* h, int32_t B, int32_t heads, int32_t S, double tau_low,
                             double tau_high, int32_t* tier, int32_t* idx, int32_t* counts, ee_stream_t stream) {
    if (eng == nullptr || h == nullptr || tier == nullptr || idx == nullptr || counts == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (B < 0 || S < 0 || heads <= 0 || (int64_t)B * S > 0x7fffffff)
        return fail(EE_ERR_INVALID_ARG, "bad shape (B, S >= 0, heads > 0, B * S < 2^31)");
    if (!aligned(h, 4) || !aligned(tier, 4) || !aligned(idx, 4) || !aligned(counts, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    EeRouteArgs a{h, tier, idx, counts, (int64_t)B * S, tau_low, tau_high, heads, S > 0 ? S : 1};
    if (heads == 1) return launch(eng, "eek_route", 1, 1, 1024, a, stream);
    // the per-row head means and tiers over the whole grid, then the partition
    if (a.rows > 0) {
        const int rc = launch(eng, "eek_route_heads_tier", cdiv(a.rows, EE_BLOCK), 1, EE_BLOCK, a, stream);
        if (rc != EE_OK) return rc;
    }
    a.heads = 0;
    return launch(eng, "eek_route", 1, 1, 1024, a, stream);
}

EE_EXPORT int ee_row_copy(ee_engine* eng, const void* src, int64_t ld_src_bytes, void* dst, int64_t ld_dst_bytes,
                          int64_t rows, int64_t row_bytes, const int32_t* idx, const int32_t* counts, int32_t tier,
                          int32_t scatter, ee_stream_t stream) {
    if (eng == nullptr || src == nullptr || dst == nullptr) return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (rows < 0 || row_bytes < 0 || ld_src_bytes < row_bytes || ld_dst_bytes < row_bytes)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (scatter != 0 && scatter != 1) return fail(EE_ERR_INVALID_ARG, "scatter must be 0 or 1");
    if (counts != nullptr && (tier < 0 || tier > 2)) return fail(EE_ERR_INVALID_ARG, "tier must be 0, 1 or 2");
    if (!aligned(idx, 4) || !aligned(counts, 4)) return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (rows == 0 || row_bytes == 0) return EE_OK;
    EeRowCopyArgs a{(const uint8_t*)src, (uint8_t*)dst, idx, counts, rows, row_bytes, ld_src_bytes, ld_dst_bytes,
                    counts ? tier : 0, scatter};
    return launch(eng, "eek_row_copy", cdiv(rows, 4), 1, EE_BLOCK, a, stream);
}

static int routed_impl(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                       const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                       const void* b_f16, const float* b_scale, void* c, int64_t ldc, void* ws_codes,
                       float* ws_scale, int sw, ee_stream_t stream, bool prequant = false) {
    if (eng == nullptr || x == nullptr || idx == nullptr || counts == nullptr || b_i8 == nullptr ||
        b_f8 == nullptr || b_f16 == nullptr || b_scale == nullptr || c == nullptr || ws_codes == nullptr ||
        ws_scale == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (M < 0 || K <= 0 || N <= 0 || ld_x < K || ldc < (sw ? N / 2 : N))
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (sw && (K % 128 != 0 || N % 64 != 0 || ldc % 8 != 0 || !aligned(c, 16)))
        return fail(EE_ERR_UNSUPPORTED, "SwiGLU routed linear needs K % 128 == 0, N % 64 == 0, ld_act % 8 == 0 "
                                        "and a 16-byte aligned act");
    // The GEMM contracts, checked here so that no launch of the sequence can fail half way.
    if (K % 16 != 0 || (ld_x * 2) % 16 != 0 || N % 4 != 0 || ldc % 4 != 0)
        return fail(EE_ERR_UNSUPPORTED, "routed linear needs K % 16 == 0, ld_x % 8 == 0, N % 4 == 0, ldc % 4 == 0");
    if (!aligned(x, 16) || !aligned(b_i8, 16) || !aligned(b_f8, 16) || !aligned(b_f16, 16) || !aligned(c, 8) ||
        !aligned(ws_codes, 16) || !aligned(ws_scale, 4) || !aligned(b_scale, 16) || !aligned(idx, 4) ||
        !aligned(counts, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (prequant && K % 128 != 0)
        return fail(EE_ERR_UNSUPPORTED, "the routed GEMM on prepared codes needs K % 128 == 0");
    if (M == 0) return EE_OK;
    int rc;
    if (prequant || (K % 128 == 0 && !opt(eng, "routed_unfused"))) {
        // Two launches: one quantiser for the INT8 and FP8 slots, then the three
        // tier GEMMs as one grid (eek_gemm_routed), scattering rows through idx.
        EeQuantArgs qa{(const uint16_t*)x, ws_codes, ws_scale, idx, counts, M, K, ld_x, K, EE_QUANT_ROUTED_I8_F8, 0,
                       nullptr, 0};
        if (!prequant && (rc = launch_quant(eng, qa, stream))) return rc;
        EeRoutedGemmArgs ra{};
        ra.t[0] = EeGemmArgs{ws_codes, b_i8, (uint16_t*)c, nullptr, ws_scale, b_scale, nullptr, idx, counts,
                             K, K, ldc, M, N, K, EE_TIER_INT8, sw};
        ra.t[1] = EeGemmArgs{ws_codes, b_f8, (uint16_t*)c, nullptr, ws_scale, b_scale, nullptr, idx, counts,
                             K, K, ldc, M, N, K, EE_TIER_FP8, sw};
        ra.t[2] = EeGemmArgs{x, b_f16, (uint16_t*)c, nullptr, nullptr, nullptr, idx, idx, counts,
                             ld_x, K, ldc, M, N, K, EE_TIER_FP16, sw};
        ra.mt_max = (int32_t)cdiv(M, 128) + 2;
        ra.f16_w8 = opt(eng, "gemm_variant") == 2;   // the FP16 pipeline ee_gemm picks (same f32 order)
        const int64_t slots = (int64_t)ra.mt_max * cdiv(N, 128);
        // Large grids: the 256 x 256-tile routed kernel (same K order in every tier).
        // Its DMA addresses rows from the operands' starts with 32-bit offsets.
        const int64_t tile_opt = opt(eng, "gemm_tile");
        const bool off32 = std::max<int64_t>((int64_t)M * ld_x * 2, (int64_t)M * K) + 2 * K < (int64_t(1) << 32) &&
                           255 * 2 * (int64_t)K + 2 * K < (int64_t(1) << 32);
        // Automatic choice: 256 x 256 tiles where they take fewer rounds of the CUs
        // at the cost of a round, ~2.1x that of a 128 x 128 round for 4x the work
        // (measured at K = 2048..5632: INT8 15 against 31 us at K = 2048, 31 against
        // 60 at K = 5632).  Tile counts take one partial M-tile beside the full ones
        // (the tiers' row counts are on the device).  Same bits either way.  Measured
        // on a 20/40/40 % tier mix, 128 tiles against 256: 1024 x 4096 x 4096 47 against
        // 59 us, 2048 x 5632 x 2048 60 against 82, 128 x 2048 x 11264 SwiGLU 31 against
        // 34 (all INT8: 23 / 47, 30 / 60, 12 / 34).
        const int64_t cu = std::max(1, eng->cus);
        const int64_t r128 = cdiv((cdiv(M, 128) + 1) * cdiv(N, 128), cu);
        const int64_t r256 = cdiv((cdiv(M, 256) + 1) * cdiv(N, 256), cu);
        const bool big = 10 * r128 > 21 * r256;
        if (!ra.f16_w8 && tile_opt != 128 && off32 && (tile_opt == 256 || big)) {
            // (256 x 256 tiles unless option gemm_tile_n = 128: the tiers' row counts, which
            // decide the rounds, are on the device)
            std::string n256 = opt(eng, "gemm_tile_n") == 128 ? "eek_gemm256n128_routed" : "eek_gemm256_routed";
            // the four-wave routed grid (same deal, same bits) where every tier's tiles
            // have at least two K stages; option gemm_waves = 8 keeps the 8-wave one
            if (opt(eng, "gemm_tile_n") != 128 && opt(eng, "gemm_waves") != 8 && K >= 256) n256 = "eek_gemm4w_routed";
            if (sw) n256 += "_swiglu";
            const Kernel* k256 = find_kernel(eng, n256);
            if (k256 != nullptr) {
                const int64_t g256 = eng->cus >= 8 ? (eng->cus & ~7) : std::max(1, eng->cus);
                const int64_t pv = opt(eng, "gemm_persist");
                return launch(eng, n256, pv >= 2 ? pv : g256, 1, k256->block, ra, stream);
            }
        }
        const int64_t pg = ra.f16_w8 ? persist_grid(eng, slots) : 0;   // its W8A16 tiles run on Gemm8
        // FP16 tiles as 128 x 64 halves where the grid then fits one round of the CUs or
        // the whole-tile grid takes one to two rounds (decided in the kernel from the
        // tier counts): possible only where one M-tile per 128 rows takes at most two
        // rounds.  The grid then holds the halves' M-tile slots too.
        int64_t grid = pg > 0 ? pg : slots;
        if (pg == 0 && !sw && !ra.f16_w8 && cdiv(M, 128) * cdiv(N, 128) <= 2 * (int64_t)eng->cus) {
            ra.mt_max = (int32_t)(2 * cdiv(M, 128) + 2);
            ra.f16_half_cus = eng->cus;
            grid = (int64_t)ra.mt_max * cdiv(N, 128);
        }
        std::string rname = pg > 0 ? "eek_gemm_routed_persist" : "eek_gemm_routed";
        if (sw) rname += "_swiglu";
        const Kernel* k = find_kernel(eng, rname);
        return launch(eng, rname, grid, 1, k ? k->block : EE_BLOCK, ra, stream);
    }
    // Any K (a multiple of 16): five launches, each tier's quantiser and GEMM.
    // INT8 rows: quantise into partition slots, GEMM, scatter.
    if ((rc = ee_quant_act(eng, x, M, K, ld_x, EE_QUANT_I8_DISPATCH, ws_codes, K, ws_scale, idx, counts,
                           EE_TIER_INT8, stream)))
        return rc;
    if ((rc = gemm_impl(eng, EE_GEMM_I8, ws_codes, K, b_i8, K, c, ldc, ws_scale, b_scale, M, N, K, nullptr, idx,
                        counts, EE_TIER_INT8, nullptr, sw, stream)))
        return rc;
    // FP8 rows.
    if ((rc = ee_quant_act(eng, x, M, K, ld_x, EE_QUANT_F8_ROW, ws_codes, K, ws_scale, idx, counts, EE_TIER_FP8,
                           stream)))
        return rc;
    if ((rc = gemm_impl(eng, EE_GEMM_F8, ws_codes, K, b_f8, K, c, ldc, ws_scale, b_scale, M, N, K, nullptr, idx,
                        counts, EE_TIER_FP8, nullptr, sw, stream)))
        return rc;
    // FP16 (W8A16) rows: gather straight from x.
    return gemm_impl(eng, EE_GEMM_F16, x, ld_x, b_f16, K, c, ldc, nullptr, nullptr, M, N, K, idx, idx, counts,
                     EE_TIER_FP16, nullptr, sw, stream);
}

EE_EXPORT int ee_routed_linear(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                               const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                               const void* b_f16, const float* b_scale, void* c, int64_t ldc, void* ws_codes,
                               float* ws_scale, ee_stream_t stream) {
    return routed_impl(eng, x, ld_x, M, K, N, idx, counts, b_i8, b_f8, b_f16, b_scale, c, ldc, ws_codes, ws_scale, 0,
                       stream);
}

EE_EXPORT int ee_routed_linear_swiglu(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                                      const int32_t* idx, const int32_t* counts, const int8_t* b_i8,
                                      const uint8_t* b_f8, const void* b_f16, const float* b_scale, void* act,
                                      int64_t ld_act, void* ws_codes, float* ws_scale, ee_stream_t stream) {
    return routed_impl(eng, x, ld_x, M, K, N, idx, counts, b_i8, b_f8, b_f16, b_scale, act, ld_act, ws_codes,
                       ws_scale, 1, stream);
}

EE_EXPORT int ee_routed_linear_noalloc(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                                       const int32_t* idx, const int32_t* counts, const int8_t* b_i8,
                                       const uint8_t* b_f8, const void* b_f16, const float* b_scale, void* c,
                                       int64_t ldc, ee_stream_t stream) {
    if (eng == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (M < 0 || K <= 0) return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (M > EE_NOALLOC_MAX_ROWS || (int64_t)M * K > EE_NOALLOC_MAX_CODE_BYTES)
        return fail(EE_ERR_UNSUPPORTED, "ee_routed_linear_noalloc holds at most " +
                                            std::to_string(EE_NOALLOC_MAX_ROWS) + " rows and " +
                                            std::to_string(EE_NOALLOC_MAX_CODE_BYTES) + " bytes of codes (M * K); got M = " +
                                            std::to_string(M) + ", K = " + std::to_string(K));
    if (eng->scratch == nullptr)
        return fail(EE_ERR_HIP, std::string("no-alloc workspace unavailable: hipGetSymbolAddress failed: ") +
                                    hipGetErrorString((hipError_t)eng->scratch_rc));
    uint8_t* codes = (uint8_t*)eng->scratch;
    float* scales = (float*)(codes + EE_NOALLOC_MAX_CODE_BYTES);
    return routed_impl(eng, x, ld_x, M, K, N, idx, counts, b_i8, b_f8, b_f16, b_scale, c, ldc, codes, scales, 0,
                       stream);
}

EE_EXPORT int ee_routed_gemm(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                             const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                             const void* b_f16, const float* b_scale, void* c, int64_t ldc, const void* codes,
                             const float* scale, ee_stream_t stream) {
    return routed_impl(eng, x, ld_x, M, K, N, idx, counts, b_i8, b_f8, b_f16, b_scale, c, ldc, (void*)codes,
                       (float*)scale, 0, stream, true);
}

EE_EXPORT int ee_routed_gemm_swiglu(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                                    const int32_t* idx, const int32_t* counts, const int8_t* b_i8,
                                    const uint8_t* b_f8, const void* b_f16, const float* b_scale, void* act,
                                    int64_t ld_act, const void* codes, const float* scale, ee_stream_t stream) {
    return routed_impl(eng, x, ld_x, M, K, N, idx, counts, b_i8, b_f8, b_f16, b_scale, act, ld_act, (void*)codes,
                       (float*)scale, 1, stream, true);
}

EE_EXPORT int ee_interleave_gate_up(ee_engine* eng, const void* src, int64_t ld_src_bytes, void* dst,
                                    int64_t ld_dst_bytes, int64_t F, int64_t row_bytes, ee_stream_t stream) {
    if (eng == nullptr || src == nullptr || dst == nullptr) return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (F < 0 || row_bytes < 0 || ld_src_bytes < row_bytes || ld_dst_bytes < row_bytes)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (F % 32 != 0 || row_bytes % 4 != 0 || ld_src_bytes % 4 != 0 || ld_dst_bytes % 4 != 0 || !aligned(src, 4) ||
        !aligned(dst, 4))
        return fail(EE_ERR_UNSUPPORTED, "interleave needs F % 32 == 0 and 4-byte aligned rows");
    if (src == dst) return fail(EE_ERR_INVALID_ARG, "interleave cannot run in place");
    if (F == 0 || row_bytes == 0) return EE_OK;
    EeInterleaveArgs a{(const uint8_t*)src, (uint8_t*)dst, F, row_bytes, ld_src_bytes, ld_dst_bytes};
    const int64_t g = std::min<int64_t>(cdiv(2 * F * (row_bytes / 4), EE_BLOCK), 16384);
    return launch(eng, "eek_interleave_rows", g, 1, EE_BLOCK, a, stream);
}

// ------------------------------------------------------------ CubinEngine counterpart

// ============================================================================ fused MLP

// interleave = 1: gu holds gate and up in alternating blocks of 32 columns (the SwiGLU weight layout).
static int silu_mul_impl(ee_engine* eng, const void* gu, int64_t ld_gu, void* act, int64_t ld_act, int64_t M,
                         int64_t F, int32_t interleave, ee_stream_t stream) {
    if (eng == nullptr || gu == nullptr || act == nullptr) return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (interleave && F % 32 != 0) return fail(EE_ERR_UNSUPPORTED, "interleaved gate|up needs F % 32 == 0");
    if (M < 0 || F <= 0 || ld_gu < 2 * F || ld_act < F) return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (!aligned(gu, 2) || !aligned(act, 2)) return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (M == 0) return EE_OK;
    const int32_t vec = F % 8 == 0 && ld_gu % 8 == 0 && ld_act % 8 == 0 && aligned(gu, 16) && aligned(act, 16);
    EeSiluMulArgs a{(const uint16_t*)gu, (uint16_t*)act, M, F, ld_gu, ld_act, vec, interleave};
    const int64_t work = vec ? M * (F / 8) : M * F;
    const int64_t g = std::min<int64_t>(cdiv(work, EE_BLOCK), 16384);
    return launch(eng, "eek_silu_mul", g, 1, EE_BLOCK, a, stream);
}

EE_EXPORT int ee_silu_mul(ee_engine* eng, const void* gu, int64_t ld_gu, void* act, int64_t ld_act, int64_t M,
                          int64_t F, ee_stream_t stream) {
    return silu_mul_impl(eng, gu, ld_gu, act, ld_act, M, F, 0, stream);
}

static int rmsnorm_args(ee_engine* eng, const void* x, int64_t ld_x, const void* y, int64_t ld_y, const void* w,
                        void* x_out, int64_t ld_xo, void* n_out, int64_t ld_n, int64_t T, int64_t D, float eps,
                        EeRmsNormArgs& a, const char*& name) {
    if (eng == nullptr || x == nullptr || w == nullptr || n_out == nullptr || (y != nullptr && x_out == nullptr))
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (T < 0 || D <= 0 || ld_x < D || ld_n < D || (y != nullptr && (ld_y < D || ld_xo < D)))
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (D % 8 != 0 || D > 4096 || ld_x % 8 != 0 || ld_n % 8 != 0 || (y != nullptr && (ld_y % 8 != 0 || ld_xo % 8 != 0)))
        return fail(EE_ERR_UNSUPPORTED, "add_rmsnorm needs D % 8 == 0, D <= 4096 and strides that are multiples of 8");
    if (!aligned(x, 16) || !aligned(y, 16) || !aligned(w, 16) || !aligned(x_out, 16) || !aligned(n_out, 16))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer (16 B)");
    a = EeRmsNormArgs{(const uint16_t*)x, (const uint16_t*)y, (const uint16_t*)w, (uint16_t*)x_out, (uint16_t*)n_out,
                      T, D, ld_x, ld_y, ld_xo, ld_n, eps, 1.0f / (float)D};
    const int64_t nc = cdiv(D / 8, 64);                // 16-byte chunks per lane
    name = nc <= 1 ? "c1" : nc <= 2 ? "c2" : nc <= 4 ? "c4" : "c8";
    return EE_OK;
}

EE_EXPORT int ee_add_rmsnorm(ee_engine* eng, const void* x, int64_t ld_x, const void* y, int64_t ld_y,
                             const void* w, void* x_out, int64_t ld_xo, void* n_out, int64_t ld_n, int64_t T,
                             int64_t D, float eps, ee_stream_t stream) {
    EeRmsNormArgs a;
    const char* nc;
    if (int rc = rmsnorm_args(eng, x, ld_x, y, ld_y, w, x_out, ld_xo, n_out, ld_n, T, D, eps, a, nc)) return rc;
    if (T == 0) return EE_OK;
    return launch(eng, std::string("eek_add_rmsnorm_") + nc, cdiv(T, EE_BLOCK / 64), 1, EE_BLOCK, a, stream);
}

EE_EXPORT int ee_add_rmsnorm_route(ee_engine* eng, const void* x, int64_t ld_x, const void* y, int64_t ld_y,
                                   const void* w, void* x_out, int64_t ld_xo, void* n_out, int64_t ld_n, int64_t T,
                                   int64_t D, float eps, const int32_t* idx, const int32_t* counts, void* codes,
                                   int64_t ld_c, float* scale, ee_stream_t stream) {
    EeRmsNormArgs a;
    const char* nc;
    if (int rc = rmsnorm_args(eng, x, ld_x, y, ld_y, w, x_out, ld_xo, n_out, ld_n, T, D, eps, a, nc)) return rc;
    if (idx == nullptr || counts == nullptr || codes == nullptr || scale == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (ld_c < D || ld_c % 8 != 0) return fail(EE_ERR_INVALID_ARG, "bad codes stride (ld_c >= D, a multiple of 8)");
    if (!aligned(codes, 8) || !aligned(scale, 4) || !aligned(idx, 4) || !aligned(counts, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer");
    if (T == 0) return EE_OK;
    EeRmsNormRouteArgs ra{a, idx, counts, (uint8_t*)codes, scale, ld_c};
    return launch(eng, std::string("eek_add_rmsnorm_route_") + nc, cdiv(T, EE_BLOCK / 64), 1, EE_BLOCK, ra, stream);
}

static int qkv_rope_impl(ee_engine* eng, const void* qkv, int64_t ld, const void* cos_t, const void* sin_t,
                         void* q, void* k, void* v, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d,
                         float q_scale, int v_t, ee_stream_t stream) {
    if (eng == nullptr || qkv == nullptr || cos_t == nullptr || sin_t == nullptr || q == nullptr || k == nullptr ||
        v == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (B < 0 || S < 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || ld < (int64_t)(Hq + 2 * Hkv) * d)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (d % 16 != 0 || ld % 8 != 0) return fail(EE_ERR_UNSUPPORTED, "qkv_rope needs d % 16 == 0 and ld % 8 == 0");
    if (v_t && S % 16 != 0) return fail(EE_ERR_UNSUPPORTED, "the transposed v layout needs S % 16 == 0");
    if (!aligned(qkv, 16) || !aligned(cos_t, 16) || !aligned(sin_t, 16) || !aligned(q, 16) || !aligned(k, 16) ||
        !aligned(v, 16))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer (16 B)");
    const int64_t T = (int64_t)B * S;
    if (T == 0) return EE_OK;
    EeQkvRopeArgs a{(const uint16_t*)qkv, (const uint16_t*)cos_t, (const uint16_t*)sin_t, (uint16_t*)q, (uint16_t*)k,
                    (uint16_t*)v, ld, B, S, Hq, Hkv, d, q_scale, v_t};
    const int64_t work = T * (Hq + Hkv) * (d / 16) + (v_t ? T / 16 : T) * Hkv * (d / 8);
    if (work >= (int64_t(1) << 31)) return fail(EE_ERR_UNSUPPORTED, "qkv_rope: more than 2^31 work items");
    return launch(eng, "eek_qkv_rope", std::min<int64_t>(cdiv(work, EE_BLOCK), 16384), 1, EE_BLOCK, a, stream);
}

EE_EXPORT int ee_qkv_rope(ee_engine* eng, const void* qkv, int64_t ld, const void* cos_t, const void* sin_t,
                          void* q, void* k, void* v, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d,
                          float q_scale, ee_stream_t stream) {
    return qkv_rope_impl(eng, qkv, ld, cos_t, sin_t, q, k, v, B, S, Hq, Hkv, d, q_scale, 0, stream);
}

EE_EXPORT int ee_qkv_rope_vt(ee_engine* eng, const void* qkv, int64_t ld, const void* cos_t, const void* sin_t,
                             void* q, void* k, void* vt, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d,
                             float q_scale, ee_stream_t stream) {
    return qkv_rope_impl(eng, qkv, ld, cos_t, sin_t, q, k, vt, B, S, Hq, Hkv, d, q_scale, 1, stream);
}

EE_EXPORT int ee_attention_causal(ee_engine* eng, const void* q, const void* k, const void* vt, void* out,
                                  int64_t ld_out, float* h, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d,
                                  ee_stream_t stream) {
    if (eng == nullptr || q == nullptr || k == nullptr || vt == nullptr || out == nullptr || h == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (B < 0 || S < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || ld_out < (int64_t)Hq * d)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride (Hq must be a multiple of Hkv, ld_out >= Hq * d)");
    if (d != 64 || S % 64 != 0 || ld_out % 8 != 0 || (Hq / Hkv) % 2 != 0)
        return fail(EE_ERR_UNSUPPORTED, "the fused attention needs head_dim 64, S % 64 == 0, ld_out % 8 == 0 and "
                                        "an even number of query heads per kv head");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(vt, 16) || !aligned(out, 16) || !aligned(h, 4))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer (q, k, vt, out: 16 B; h: 4 B)");
    if ((int64_t)B * S == 0) return EE_OK;
    const int G = Hq / Hkv;
    const int W = G % 4 == 0 ? 4 : 2;
    EeAttnArgs a{(const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)vt, (uint16_t*)out, h, ld_out, B, S, Hq,
                 Hkv, W};
    return launch(eng, "eek_attn_causal_d64_w" + std::to_string(W), (int64_t)B * (Hq / W) * (S / 64), 1, 64 * W, a,
                  stream);
}

EE_EXPORT int ee_mlp_prepare(ee_engine* eng, const void* gate_w, const void* up_w, const void* down_w, int64_t H,
                             int64_t F, int64_t ld_gate, int64_t ld_up, int64_t ld_down, int8_t* gu_i8,
                             uint8_t* gu_f8, void* gu_f16, float* gu_scale, int8_t* dn_i8, uint8_t* dn_f8,
                             void* dn_f16, float* dn_scale, ee_stream_t stream) {
    if (eng == nullptr || gate_w == nullptr || up_w == nullptr || down_w == nullptr || gu_i8 == nullptr ||
        gu_f8 == nullptr || gu_f16 == nullptr || gu_scale == nullptr || dn_i8 == nullptr || dn_f8 == nullptr ||
        dn_f16 == nullptr || dn_scale == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (H <= 0 || F <= 0 || ld_gate < H || ld_up < H || ld_down < F)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (F % 32 != 0 || H % 4 != 0) return fail(EE_ERR_UNSUPPORTED, "the MLP engine needs F % 32 == 0, H % 4 == 0");
    int rc;
    // gate|up: one [2F, H] operand, gate and up rows interleaved in blocks of 32 (the SwiGLU
    // epilogue's pairing).  Per-row scales are per output channel, so quantising the halves
    // separately and permuting rows equals quantising the permuted operand.  The FP8 and
    // W8A16 buffers hold the unpermuted codes and scales until they are packed.
    uint8_t* codes_tmp = gu_f8;
    float* scale_tmp = (float*)gu_f16;
    if ((rc = ee_quant_weight_i8(eng, gate_w, F, H, ld_gate, (int8_t*)codes_tmp, H, scale_tmp, stream))) return rc;
    if ((rc = ee_quant_weight_i8(eng, up_w, F, H, ld_up, (int8_t*)codes_tmp + F * H, H, scale_tmp + F, stream)))
        return rc;
    if ((rc = ee_interleave_gate_up(eng, codes_tmp, H, gu_i8, H, F, H, stream))) return rc;
    if ((rc = ee_interleave_gate_up(eng, scale_tmp, 4, gu_scale, 4, F, 4, stream))) return rc;
    if ((rc = ee_pack_b_f8(eng, gu_i8, 2 * F, H, H, gu_f8, H, stream))) return rc;
    if ((rc = ee_pack_b_f16(eng, gu_i8, gu_scale, 2 * F, H, H, gu_f16, H, stream))) return rc;
    if ((rc = ee_quant_weight_i8(eng, down_w, H, F, ld_down, dn_i8, F, dn_scale, stream))) return rc;
    if ((rc = ee_pack_b_f8(eng, dn_i8, H, F, F, dn_f8, F, stream))) return rc;
    return ee_pack_b_f16(eng, dn_i8, dn_scale, H, F, F, dn_f16, F, stream);
}

namespace {
// Workspace carve-up of ee_mlp_forward: each region 256-byte aligned.
struct MlpWs {
    uint8_t* codes; float* scale; uint16_t* gu; uint16_t* act; int32_t* tier; int32_t* idx; int32_t* counts;
    int64_t bytes;
};
MlpWs mlp_ws(void* base, int64_t M, int64_t H, int64_t F, bool routed) {
    auto up = [](int64_t v) { return (v + 255) & ~int64_t(255); };
    MlpWs w{};
    int64_t o = 0;
    uint8_t* b = (uint8_t*)base;
    w.codes = b + o; o = up(o + M * std::max(H, F));
    w.scale = (float*)(b + o); o = up(o + M * 4);
    w.gu = (uint16_t*)(b + o); o = up(o + M * 2 * F * 2);
    w.act = (uint16_t*)(b + o); o = up(o + M * F * 2);
    if (routed) {
        w.tier = (int32_t*)(b + o); o = up(o + M * 4);
        w.idx = (int32_t*)(b + o); o = up(o + M * 4);
        w.counts = (int32_t*)(b + o); o = up(o + 16);
    }
    w.bytes = o;
    return w;
}
}  // namespace

EE_EXPORT int64_t ee_mlp_workspace_bytes(int64_t M, int64_t H, int64_t F, int32_t routed) {
    if (M < 0 || H <= 0 || F <= 0) return -1;
    return mlp_ws(nullptr, M, H, F, routed != 0).bytes;
}

EE_EXPORT int ee_mlp_forward(ee_engine* eng, const void* x, int64_t ld_x, int64_t M, int64_t H, int64_t F,
                             const int8_t* gu_i8, const uint8_t* gu_f8, const void* gu_f16, const float* gu_scale,
                             const int8_t* dn_i8, const uint8_t* dn_f8, const void* dn_f16, const float* dn_scale,
                             double entropy, const float* h_rows, double tau_low, double tau_high, void* out,
                             int64_t ldo, void* workspace, int64_t ws_bytes, ee_stream_t stream) {
    if (eng == nullptr || x == nullptr || out == nullptr || workspace == nullptr || gu_i8 == nullptr ||
        gu_f8 == nullptr || gu_f16 == nullptr || gu_scale == nullptr || dn_i8 == nullptr || dn_f8 == nullptr ||
        dn_f16 == nullptr || dn_scale == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (M < 0 || M > 0x7fffffff || H <= 0 || F <= 0 || ld_x < H || ldo < H)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (H % 16 != 0 || F % 32 != 0 || ld_x % 8 != 0 || ldo % 4 != 0)
        return fail(EE_ERR_UNSUPPORTED, "fused MLP needs H % 16 == 0, F % 32 == 0, ld_x % 8 == 0, ldo % 4 == 0");
    if (!aligned(x, 16) || !aligned(out, 8) || !aligned(workspace, 256))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer (x 16 B, out 8 B, workspace 256 B)");
    const MlpWs w = mlp_ws(workspace, M, H, F, h_rows != nullptr);
    if (ws_bytes < w.bytes)
        return fail(EE_ERR_INVALID_ARG, "workspace too small: need " + std::to_string(w.bytes) + " bytes");
    if (M == 0) return EE_OK;
    const int32_t m = (int32_t)M, h = (int32_t)H, f = (int32_t)F;
    int rc;
    if (h_rows != nullptr) {
        // one tier per row: route, gate|up routed linear, activation, down routed linear
        if ((rc = ee_route(eng, h_rows, M, tau_low, tau_high, w.tier, w.idx, w.counts, stream))) return rc;
        if (H % 128 == 0) {                           // gate|up GEMMs write silu(gate) * up directly
            if ((rc = routed_impl(eng, x, ld_x, m, h, 2 * f, w.idx, w.counts, gu_i8, gu_f8, gu_f16, gu_scale, w.act,
                                  F, w.codes, w.scale, 1, stream)))
                return rc;
        } else {
            if ((rc = ee_routed_linear(eng, x, ld_x, m, h, 2 * f, w.idx, w.counts, gu_i8, gu_f8, gu_f16, gu_scale,
                                       w.gu, 2 * F, w.codes, w.scale, stream)))
                return rc;
            if ((rc = silu_mul_impl(eng, w.gu, 2 * F, w.act, F, M, F, 1, stream))) return rc;
        }
        return ee_routed_linear(eng, w.act, F, m, f, h, w.idx, w.counts, dn_i8, dn_f8, dn_f16, dn_scale, out, ldo,
                                w.codes, w.scale, stream);
    }
    // one tier for the call, by the dispatcher's strict comparisons (EE/python/dispatch.py:74-79)
    const int tier = entropy < tau_low ? EE_TIER_INT8 : (entropy < tau_high ? EE_TIER_FP8 : EE_TIER_FP16);
    if (tier == EE_TIER_FP16) {
        const int sw = H % 64 == 0;                   // the pipelined W8A16 kernels: K * 2 % 128 == 0
        if ((rc = gemm_impl(eng, EE_GEMM_F16, x, ld_x, gu_f16, H, sw ? (void*)w.act : (void*)w.gu, sw ? F : 2 * F,
                            nullptr, nullptr, m, 2 * f, h, nullptr, nullptr, nullptr, 0, nullptr, sw, stream)))
            return rc;
        if (!sw && (rc = silu_mul_impl(eng, w.gu, 2 * F, w.act, F, M, F, 1, stream))) return rc;
        return ee_gemm(eng, EE_GEMM_F16, w.act, F, dn_f16, F, out, ldo, nullptr, nullptr, m, h, f, nullptr, nullptr,
                       nullptr, 0, nullptr, stream);
    }
    const int32_t qmode = tier == EE_TIER_INT8 ? EE_QUANT_I8_DISPATCH : EE_QUANT_F8_ROW;
    const int32_t kind = tier == EE_TIER_INT8 ? EE_GEMM_I8 : EE_GEMM_F8;
    const void* bgu = tier == EE_TIER_INT8 ? (const void*)gu_i8 : (const void*)gu_f8;
    const void* bdn = tier == EE_TIER_INT8 ? (const void*)dn_i8 : (const void*)dn_f8;
    if ((rc = ee_quant_act(eng, x, M, H, ld_x, qmode, w.codes, H, w.scale, nullptr, nullptr, 0, stream))) return rc;
    const int sw = H % 128 == 0;                      // the pipelined 1-byte kernels: K % 128 == 0
    if ((rc = gemm_impl(eng, kind, w.codes, H, bgu, H, sw ? (void*)w.act : (void*)w.gu, sw ? F : 2 * F, w.scale,
                        gu_scale, m, 2 * f, h, nullptr, nullptr, nullptr, 0, nullptr, sw, stream)))
        return rc;
    if (!sw && (rc = silu_mul_impl(eng, w.gu, 2 * F, w.act, F, M, F, 1, stream))) return rc;
    if ((rc = ee_quant_act(eng, w.act, M, F, F, qmode, w.codes, F, w.scale, nullptr, nullptr, 0, stream))) return rc;
    return ee_gemm(eng, kind, w.codes, F, bdn, F, out, ldo, w.scale, dn_scale, m, h, f, nullptr, nullptr, nullptr, 0,
                   nullptr, stream);
}

EE_EXPORT int ee_module_engine_create(const char* code_object_path, const char* func_name, int32_t shared_mem,
                                      int32_t num_warps, int32_t block_m, int32_t block_n, ee_module_engine** out) {
    if (out == nullptr) return fail(EE_ERR_INVALID_ARG, "out must not be NULL");
    *out = nullptr;
    if (code_object_path == nullptr || func_name == nullptr)
        return fail(EE_ERR_INVALID_ARG, "code_object_path and func_name must not be NULL");
    if (num_warps <= 0 || num_warps * 64 > 1024) return fail(EE_ERR_INVALID_ARG, "num_warps must be in 1..16 (wave64)");
    if (block_m <= 0 || block_n <= 0 || shared_mem < 0) return fail(EE_ERR_INVALID_ARG, "bad tile or shared size");
    std::string bytes;
    int rc = read_file(code_object_path, bytes, "code object file");
    if (rc) return rc;
    if (bytes.size() < 4 || std::memcmp(bytes.data(), "\x7f" "ELF", 4) != 0)
        return fail(EE_ERR_IO, std::string("Not an ELF code object: ") + code_object_path);
    std::unique_ptr<ee_module_engine> me(new ee_module_engine());
    EE_HIP(hipGetDevice(&me->device), "hipGetDevice");
    EE_HIP(hipModuleLoadData(&me->module, bytes.data()), std::string("hipModuleLoadData failed for ") + code_object_path);
    hipError_t err = hipModuleGetFunction(&me->fn, me->module, func_name);
    if (err != hipSuccess) {
        (void)hipModuleUnload(me->module);
        return fail(EE_ERR_NOT_FOUND, std::string("hipModuleGetFunction failed for '") + func_name + "' in " +
                                          code_object_path + ": " + hipGetErrorString(err));
    }
    int max_threads = 0, lds = 0;
    if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, me->fn) != hipSuccess ||
        hipFuncGetAttribute(&lds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, me->fn) != hipSuccess) {
        (void)hipModuleUnload(me->module);
        return fail(EE_ERR_HIP, "hipFuncGetAttribute failed");
    }
    // The GEMM kernels assume exactly their 256-thread workgroup and 128x128 tile.
    if (num_warps * 64 != max_threads || block_m != 128 || block_n != 128) {
        (void)hipModuleUnload(me->module);
        return fail(EE_ERR_META, std::string("launch config (num_warps ") + std::to_string(num_warps) +
                                     ", BLOCK_M " + std::to_string(block_m) + ", BLOCK_N " + std::to_string(block_n) +
                                     ") does not match '" + func_name + "' (" + std::to_string(max_threads / 64) +
                                     " wave64s, 128x128 tile)");
    }
    me->func = func_name;
    me->shared_mem = shared_mem;
    me->num_warps = num_warps;
    me->block_m = block_m;
    me->block_n = block_n;
    me->static_lds = lds;
    *out = me.release();
    return EE_OK;
}

EE_EXPORT int ee_module_engine_from_metadata(const char* code_object_path, const char* meta_json_path,
                                             const char* func_name, ee_module_engine** out) {
    if (out == nullptr) return fail(EE_ERR_INVALID_ARG, "out must not be NULL");
    *out = nullptr;
    if (meta_json_path == nullptr) return fail(EE_ERR_INVALID_ARG, "meta_json_path must not be NULL");
    std::string text;
    int rc = read_file(meta_json_path, text, "meta JSON");
    if (rc) return rc;
    Json meta;
    if ((rc = parse_json(text, meta_json_path, meta))) return rc;
    int64_t shared = 0, warps = 0, bm = 0, bn = 0;
    if ((rc = json_int(meta, "shared", meta_json_path, shared))) return rc;
    if ((rc = json_int(meta, "num_warps", meta_json_path, warps))) return rc;
    if ((rc = json_int(meta, "BLOCK_M", meta_json_path, bm))) return rc;
    if ((rc = json_int(meta, "BLOCK_N", meta_json_path, bn))) return rc;
    return ee_module_engine_create(code_object_path, func_name, (int32_t)shared, (int32_t)warps, (int32_t)bm,
                                   (int32_t)bn, out);
}

EE_EXPORT int ee_module_engine_info(const ee_module_engine* me, int32_t* shared_mem, int32_t* num_warps,
                                    int32_t* block_m, int32_t* block_n) {
    if (me == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (shared_mem) *shared_mem = me->shared_mem;
    if (num_warps) *num_warps = me->num_warps;
    if (block_m) *block_m = me->block_m;
    if (block_n) *block_n = me->block_n;
    return EE_OK;
}

EE_EXPORT int ee_module_engine_forward(ee_module_engine* me, const int8_t* a, int64_t lda, const int8_t* b_nk,
                                       int64_t ldb, void* c, int64_t ldc, const float* a_scale, const float* b_scale,
                                       int32_t M, int32_t N, int32_t K, ee_stream_t stream) {
    if (me == nullptr) return fail(EE_ERR_INVALID_ARG, "engine must not be NULL");
    if (a == nullptr || b_nk == nullptr || c == nullptr || a_scale == nullptr || b_scale == nullptr)
        return fail(EE_ERR_INVALID_ARG, "NULL argument");
    if (M < 0 || N <= 0 || K <= 0 || lda < K || ldb < K || ldc < N)
        return fail(EE_ERR_INVALID_ARG, "bad shape or stride");
    if (K % 16 != 0 || lda % 16 != 0 || ldb % 16 != 0 || N % 4 != 0 || ldc % 4 != 0)
        return fail(EE_ERR_UNSUPPORTED, "need K, lda, ldb multiples of 16 and N, ldc multiples of 4");
    const bool generic = me->func.size() > 8 && me->func.compare(me->func.size() - 8, 8, "_generic") == 0;
    if (!generic && K % 128 != 0)
        return fail(EE_ERR_UNSUPPORTED, "'" + me->func + "' streams 128-byte K stages: K must be a multiple of 128 "
                                        "(the *_generic kernel takes any multiple of 16)");
    if (!aligned(a, 16) || !aligned(b_nk, 16) || !aligned(c, 8) || !aligned(a_scale, 4) || !aligned(b_scale, 16))
        return fail(EE_ERR_INVALID_ARG, "misaligned pointer (a, b, b_scale: 16 B; c: 8 B; a_scale: 4 B)");
    if (M == 0) return EE_OK;
    int rc = check_device(me->device);
    if (rc) return rc;
    EeGemmArgs g{a, b_nk, (uint16_t*)c, nullptr, a_scale, b_scale, nullptr, nullptr, nullptr, lda, ldb, ldc,
                 M, N, K, 0};
    const int64_t grid = cdiv(M, me->block_m) * cdiv(N, me->block_n);
    const int dyn = me->shared_mem > me->static_lds ? me->shared_mem - me->static_lds : 0;
    void* params[] = {&g};
    EE_HIP(hipModuleLaunchKernel(me->fn, (unsigned)grid, 1, 1, (unsigned)(me->num_warps * 64), 1, 1, (unsigned)dyn,
                                 (hipStream_t)stream, params, nullptr),
           "hipModuleLaunchKernel");
    return EE_OK;
}

EE_EXPORT int ee_module_engine_destroy(ee_module_engine* me) {
    if (me == nullptr) return EE_OK;
    int rc = EE_OK;
    if (me->module != nullptr && hipModuleUnload(me->module) != hipSuccess) rc = fail(EE_ERR_HIP, "hipModuleUnload failed");
    delete me;
    return rc;
}
