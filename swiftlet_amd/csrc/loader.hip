// Checkpoint and .qpack loading into HBM: the files an mlx-lm checkpoint
// directory or a .qpack container holds, read with pread and streamed to the
// device through two pinned staging buffers (a chunk is read from the file
// while the previous one crosses PCIe), or returned on the host as raw bytes.
//
//   checkpoint  Checkpoint (Checkpoint.swift:28-72): model.safetensors, or
//               the shards a model.safetensors.index.json maps; the
//               "quantization" block of config.json (default + per-module
//               overrides, :31-47); "language_model." names resolved as
//               :76-80 does; residentLinear (MetalShardStore.swift:67-118)
//               as one device buffer per module (codes | scales | biases).
//   qpack       Qpack.Layout / Manifest (Qpack.swift:22-46) and
//               QpackExpertReader (:168-203).  An MI355X holds every layer's
//               expert file in HBM (35B q4: 40 x 256 blobs of 1.77 MB =
//               18 GB of 288 GB), so a layer file is copied to the device
//               byte for byte and the expert matrices are addressed inside
//               the blobs: matrix m of expert e starts at
//               base + e * expertStride + section(m).offset, which is a stacked
//               swq_qlinear with expert_stride_w = expert_stride_sb = the
//               blob stride.  No repacking on load.
//
// Handles are not thread-safe (one staging pair each).  Host-side functions
// (open, info, host reads) make no HIP call.
#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "internal.hpp"
#include "json.hpp"

namespace swq {
namespace loader {

constexpr size_t kStageBytes = 16u << 20;      // per staging buffer
constexpr int64_t kMaxHeaderBytes = 256 << 20;  // a safetensors JSON header
constexpr int64_t kQpackPageAlignment = 16384;  // Qpack.pageAlignment (Qpack.swift:19)

int64_t dtype_size(const std::string &d) {
    if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E5M2" || d == "F8_E4M3") return 1;
    if (d == "I16" || d == "U16" || d == "F16" || d == "BF16") return 2;
    if (d == "I32" || d == "U32" || d == "F32") return 4;
    if (d == "I64" || d == "U64" || d == "F64") return 8;
    return 0;
}

int scales_type_of(const std::string &d) {  // MetalEngine.ScalesType (MetalEngine.swift:69-80)
    if (d == "F32") return SWQ_F32;
    if (d == "F16") return SWQ_F16;
    if (d == "BF16") return SWQ_BF16;
    return -1;
}

bool read_exact(int fd, void *dst, int64_t n, int64_t off) {
    uint8_t *p = static_cast<uint8_t *>(dst);
    while (n > 0) {
        const ssize_t r = pread(fd, p, static_cast<size_t>(std::min<int64_t>(n, 1 << 30)), off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        off += r;
        n -= r;
    }
    return true;
}

// read_exact split over up to kReadThreads threads (slices of >= 2 MiB): a
// page-cache read is a memory copy, and one thread's copy rate is below
// what the host link takes.
constexpr int kReadThreads = 4;

bool read_parallel(int fd, void *dst, int64_t n, int64_t off) {
    const int64_t slice = std::max<int64_t>(2 << 20, (n + kReadThreads - 1) / kReadThreads);
    const int parts = static_cast<int>(std::min<int64_t>(kReadThreads, (n + slice - 1) / slice));
    if (parts <= 1) return read_exact(fd, dst, n, off);
    bool ok[kReadThreads];
    std::thread th[kReadThreads];
    for (int i = 1; i < parts; ++i) {
        const int64_t b = i * slice, len = std::min(slice, n - b);
        th[i] = std::thread([&, i, b, len] { ok[i] = read_exact(fd, static_cast<uint8_t *>(dst) + b, len, off + b); });
    }
    ok[0] = read_exact(fd, dst, std::min(slice, n), off);
    bool all = ok[0];
    for (int i = 1; i < parts; ++i) {
        th[i].join();
        all = all && ok[i];
    }
    return all;
}

bool read_text(const std::string &path, std::string &out) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && st.st_size >= 0 && st.st_size <= kMaxHeaderBytes;
    if (ok) {
        out.resize(static_cast<size_t>(st.st_size));
        ok = read_exact(fd, &out[0], st.st_size, 0);
    }
    close(fd);
    return ok;
}

bool file_exists(const std::string &path) {
    struct stat st;
    return stat(path.c_str(), &st) == 0;
}

struct Tensor {
    std::string dtype;
    std::vector<int64_t> shape;
    int64_t begin = 0, nbytes = 0;  // absolute offset in its file, size
    int file = 0;
};

void fill_info(const Tensor &t, swq_tensor_info *info) {
    std::memset(info, 0, sizeof(*info));
    std::strncpy(info->dtype, t.dtype.c_str(), sizeof(info->dtype) - 1);
    info->ndim = static_cast<int32_t>(t.shape.size());
    for (size_t i = 0; i < t.shape.size() && i < SWQ_MAX_DIMS; ++i) info->shape[i] = t.shape[i];
    info->nbytes = t.nbytes;
}

// Shape from a JSON array of non-negative integers (at most SWQ_MAX_DIMS).
bool json_shape(const json::Value *v, std::vector<int64_t> &shape) {
    if (!v || v->kind != json::Value::Array || v->arr.size() > SWQ_MAX_DIMS) return false;
    shape.clear();
    for (const auto &d : v->arr) {
        if (!d.is_int() || d.i < 0) return false;
        shape.push_back(d.i);
    }
    return true;
}

int64_t elements(const std::vector<int64_t> &shape) {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d != 0 && n > (int64_t(1) << 50) / d) return -1;
        n *= d;
    }
    return n;
}

// Two pinned buffers and their copy-done events: a chunk is read into one
// while the other's copy drains.  Allocated on first use.
struct Staging {
    void *buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};

    int ensure() {
        for (int i = 0; i < 2; ++i) {
            if (!buf[i] && hipHostMalloc(&buf[i], kStageBytes, hipHostMallocDefault) != hipSuccess) {
                buf[i] = nullptr;
                return SWQ_ERR_HIP;
            }
            if (!ev[i] && hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) {
                ev[i] = nullptr;
                return SWQ_ERR_HIP;
            }
        }
        return SWQ_OK;
    }
    void release() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) hipEventDestroy(ev[i]);
            if (buf[i]) hipHostFree(buf[i]);
            ev[i] = nullptr;
            buf[i] = nullptr;
        }
    }

    // n bytes of fd at off into device memory dst, stream-ordered on s;
    // returns after the last copy has completed (the buffers are free again).
    int to_device(int fd, int64_t off, int64_t n, uint8_t *dst, hipStream_t s) {
        int st = ensure();
        if (st != SWQ_OK) return st;
        int64_t done = 0;
        int k = 0;
        used[0] = used[1] = false;
        while (done < n) {
            const int b = k & 1;
            if (used[b] && hipEventSynchronize(ev[b]) != hipSuccess) return SWQ_ERR_HIP;
            const int64_t len = std::min<int64_t>(n - done, static_cast<int64_t>(kStageBytes));
            if (!read_parallel(fd, buf[b], len, off + done)) {
                drain();
                return SWQ_ERR_IO;
            }
            if (hipMemcpyAsync(dst + done, buf[b], static_cast<size_t>(len), hipMemcpyHostToDevice, s) != hipSuccess ||
                hipEventRecord(ev[b], s) != hipSuccess) {
                drain();
                return SWQ_ERR_HIP;
            }
            used[b] = true;
            done += len;
            ++k;
        }
        return drain();
    }
    int drain() {
        int st = SWQ_OK;
        for (int i = 0; i < 2; ++i)
            if (used[i] && hipEventSynchronize(ev[i]) != hipSuccess) st = SWQ_ERR_HIP;
        used[0] = used[1] = false;
        return st;
    }
};

}  // namespace loader
}  // namespace swq

using namespace swq;
using namespace swq::loader;

// ===========================================================================
// checkpoint

struct swq_checkpoint {
    std::string dir;
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::vector<int64_t> sizes;
    std::map<std::string, Tensor> tensors;
    std::vector<const std::string *> names;  // tensors' keys, for listing
    bool has_default = false;
    int def_group = 0, def_bits = 0;
    std::map<std::string, std::pair<int, int>> overrides;  // module key -> (group, bits)
    Staging staging;

    ~swq_checkpoint() {
        staging.release();
        for (int fd : fds)
            if (fd >= 0) close(fd);
    }

    // Checkpoint.resolve (Checkpoint.swift:76-80)
    const Tensor *find(const std::string &name) const {
        auto it = tensors.find(name);
        if (it != tensors.end()) return &it->second;
        it = tensors.find("language_model." + name);
        return it == tensors.end() ? nullptr : &it->second;
    }

    // One safetensors file: an 8-byte little-endian header length, the JSON
    // header (name -> dtype, shape, data_offsets relative to the data start;
    // "__metadata__" skipped), then the data.  only: the names this file
    // must hold (from an index), or every name when null.
    int add_file(const std::string &path, const std::vector<std::string> *only) {
        const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) return SWQ_ERR_IO;
        const int index = static_cast<int>(fds.size());
        fds.push_back(fd);
        paths.push_back(path);
        struct stat st;
        if (fstat(fd, &st) != 0) return SWQ_ERR_IO;
        sizes.push_back(st.st_size);
        uint8_t len8[8];
        if (st.st_size < 8 || !read_exact(fd, len8, 8, 0)) return SWQ_ERR_FORMAT;
        uint64_t hlen = 0;
        for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | len8[i];
        if (hlen > static_cast<uint64_t>(kMaxHeaderBytes) || static_cast<int64_t>(8 + hlen) > st.st_size)
            return SWQ_ERR_FORMAT;
        std::string text(hlen, '\0');
        if (!read_exact(fd, &text[0], static_cast<int64_t>(hlen), 8)) return SWQ_ERR_IO;
        json::Value h;
        if (!json::parse(text, h) || h.kind != json::Value::Object) return SWQ_ERR_FORMAT;
        const int64_t data0 = 8 + static_cast<int64_t>(hlen);
        for (const auto &kv : h.obj) {
            if (kv.first == "__metadata__") continue;
            if (only && std::find(only->begin(), only->end(), kv.first) == only->end()) continue;
            const json::Value *dt = kv.second.get("dtype"), *off = kv.second.get("data_offsets");
            Tensor t;
            if (!dt || dt->kind != json::Value::String || !json_shape(kv.second.get("shape"), t.shape))
                return SWQ_ERR_FORMAT;
            if (!off || off->kind != json::Value::Array || off->arr.size() != 2 || !off->arr[0].is_int() ||
                !off->arr[1].is_int())
                return SWQ_ERR_FORMAT;
            const int64_t b = off->arr[0].i, e = off->arr[1].i, es = dtype_size(dt->s), ne = elements(t.shape);
            if (b < 0 || e < b || data0 + e > st.st_size || es == 0 || ne < 0 || ne * es != e - b)
                return SWQ_ERR_FORMAT;
            t.dtype = dt->s;
            t.begin = data0 + b;
            t.nbytes = e - b;
            t.file = index;
            tensors[kv.first] = t;
        }
        return SWQ_OK;
    }

    int open_dir(const std::string &d) {
        dir = d;
        // quantization spec (Checkpoint.swift:31-47)
        std::string cfg_text;
        if (read_text(dir + "/config.json", cfg_text)) {
            json::Value cfg;
            if (!json::parse(cfg_text, cfg)) return SWQ_ERR_FORMAT;
            const json::Value *q = cfg.get("quantization");
            if (q && q->kind == json::Value::Object) {
                const json::Value *g = q->get("group_size"), *b = q->get("bits");
                if (g && b && g->is_int() && b->is_int()) {
                    has_default = true;
                    def_group = static_cast<int>(g->i);
                    def_bits = static_cast<int>(b->i);
                }
                for (const auto &kv : q->obj) {
                    const json::Value *sg = kv.second.get("group_size"), *sb = kv.second.get("bits");
                    if (sg && sb && sg->is_int() && sb->is_int())
                        overrides[kv.first] = {static_cast<int>(sg->i), static_cast<int>(sb->i)};
                }
            }
        }
        // files (Checkpoint.swift:50-71)
        const std::string index = dir + "/model.safetensors.index.json";
        int st = SWQ_OK;
        if (file_exists(index)) {
            std::string text;
            json::Value ix;
            if (!read_text(index, text) || !json::parse(text, ix)) return SWQ_ERR_FORMAT;
            const json::Value *wm = ix.get("weight_map");
            if (!wm || wm->kind != json::Value::Object) return SWQ_ERR_FORMAT;
            std::map<std::string, std::vector<std::string>> by_file;
            for (const auto &kv : wm->obj) {
                if (kv.second.kind != json::Value::String || kv.second.s.find('/') != std::string::npos)
                    return SWQ_ERR_FORMAT;
                by_file[kv.second.s].push_back(kv.first);
            }
            for (const auto &f : by_file) {
                if ((st = add_file(dir + "/" + f.first, &f.second)) != SWQ_OK) return st;
                for (const auto &name : f.second)
                    if (tensors.find(name) == tensors.end()) return SWQ_ERR_FORMAT;  // mapped but absent
            }
        } else {
            if ((st = add_file(dir + "/model.safetensors", nullptr)) != SWQ_OK) return st;
        }
        for (const auto &kv : tensors) names.push_back(&kv.first);
        return SWQ_OK;
    }

    // Checkpoint.quantSpec (Checkpoint.swift:111-120).  The reference returns
    // the first matching override in dictionary order; this takes the
    // longest (most specific) matching key, the same spec whenever one key
    // matches.
    bool quant(const std::string &path, int &group, int &bits) const {
        if (!find(path + ".scales")) return false;
        size_t best = 0;
        bool found = false;
        for (const auto &kv : overrides) {
            const std::string &k = kv.first;
            const bool match = (path.size() >= k.size() && path.compare(path.size() - k.size(), k.size(), k) == 0) ||
                               (k.size() >= path.size() && k.compare(k.size() - path.size(), path.size(), path) == 0);
            if (match && (!found || k.size() > best)) {
                found = true;
                best = k.size();
                group = kv.second.first;
                bits = kv.second.second;
            }
        }
        if (found) return true;
        if (!has_default) return false;
        group = def_group;
        bits = def_bits;
        return true;
    }
};

namespace {

inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// The device layout of one resident module: codes at 0, scales and biases
// each at the next 256-byte boundary.
struct LinearPlan {
    const Tensor *w, *s, *b;
    int group, bits, stype;
    int64_t s_off, b_off, total;
};

int plan_linear(const swq_checkpoint *c, const char *path, LinearPlan &p) {
    if (!c || !path) return SWQ_ERR_INVALID_ARGUMENT;
    const std::string m(path);
    p.w = c->find(m + ".weight");
    if (!p.w) return SWQ_ERR_MISSING_TENSOR;
    if (!c->quant(m, p.group, p.bits)) return c->find(m + ".scales") ? SWQ_ERR_FORMAT : SWQ_ERR_UNSUPPORTED_BITS;
    p.s = c->find(m + ".scales");
    p.b = c->find(m + ".biases");
    if (!p.s || !p.b) return SWQ_ERR_MISSING_TENSOR;
    if (p.bits != 2 && p.bits != 4 && p.bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
    if (p.w->dtype != "U32" || p.w->shape.empty()) return SWQ_ERR_FORMAT;
    p.stype = scales_type_of(p.s->dtype);
    if (p.stype < 0 || p.b->dtype != p.s->dtype) return SWQ_ERR_UNSUPPORTED_DTYPE;
    p.s_off = align256(p.w->nbytes);
    p.b_off = align256(p.s_off + p.s->nbytes);
    p.total = p.b_off + p.b->nbytes;
    return SWQ_OK;
}

}  // namespace

extern "C" int swq_checkpoint_open(const char *dir, swq_checkpoint **out) {
    if (!dir || !out) return SWQ_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    swq_checkpoint *c = new (std::nothrow) swq_checkpoint();
    if (!c) return SWQ_ERR_IO;
    int st;
    try {
        st = c->open_dir(dir);
    } catch (...) {
        st = SWQ_ERR_FORMAT;
    }
    if (st != SWQ_OK) {
        delete c;
        return st;
    }
    *out = c;
    return SWQ_OK;
}

extern "C" void swq_checkpoint_close(swq_checkpoint *c) { delete c; }

extern "C" int swq_checkpoint_tensor_count(const swq_checkpoint *c) {
    return c ? static_cast<int>(c->names.size()) : SWQ_ERR_INVALID_ARGUMENT;
}

extern "C" const char *swq_checkpoint_tensor_name(const swq_checkpoint *c, int i) {
    if (!c || i < 0 || i >= static_cast<int>(c->names.size())) return nullptr;
    return c->names[static_cast<size_t>(i)]->c_str();
}

extern "C" int swq_checkpoint_tensor(const swq_checkpoint *c, const char *name, swq_tensor_info *info) {
    if (!c || !name || !info) return SWQ_ERR_INVALID_ARGUMENT;
    const Tensor *t = c->find(name);
    if (!t) return SWQ_ERR_MISSING_TENSOR;
    fill_info(*t, info);
    return SWQ_OK;
}

extern "C" int swq_checkpoint_quant(const swq_checkpoint *c, const char *path, int *group_size, int *bits) {
    if (!c || !path || !group_size || !bits) return SWQ_ERR_INVALID_ARGUMENT;
    int g = 0, b = 0;
    if (!c->quant(path, g, b)) return SWQ_ERR_MISSING_TENSOR;
    *group_size = g;
    *bits = b;
    return SWQ_OK;
}

extern "C" int swq_checkpoint_read(const swq_checkpoint *c, const char *name, void *dst, int64_t dst_bytes) {
    if (!c || !name || !dst) return SWQ_ERR_INVALID_ARGUMENT;
    const Tensor *t = c->find(name);
    if (!t) return SWQ_ERR_MISSING_TENSOR;
    if (dst_bytes < t->nbytes) return SWQ_ERR_INVALID_ARGUMENT;
    return read_exact(c->fds[t->file], dst, t->nbytes, t->begin) ? SWQ_OK : SWQ_ERR_IO;
}

extern "C" int swq_checkpoint_load(swq_checkpoint *c, const char *name, void *dst, int64_t dst_bytes,
                                   void *stream) {
    if (!c || !name || !dst) return SWQ_ERR_INVALID_ARGUMENT;
    const Tensor *t = c->find(name);
    if (!t) return SWQ_ERR_MISSING_TENSOR;
    if (dst_bytes < t->nbytes) return SWQ_ERR_INVALID_ARGUMENT;
    return c->staging.to_device(c->fds[t->file], t->begin, t->nbytes, static_cast<uint8_t *>(dst),
                                static_cast<hipStream_t>(stream));
}

extern "C" int64_t swq_checkpoint_linear_bytes(const swq_checkpoint *c, const char *path) {
    LinearPlan p;
    const int st = plan_linear(c, path, p);
    return st == SWQ_OK ? p.total : st;
}

extern "C" int swq_checkpoint_linear(swq_checkpoint *c, const char *path, int rows_per_expert, void *dst,
                                     int64_t dst_bytes, swq_qlinear *out, void *stream) {
    if (!out || !dst || rows_per_expert < 0) return SWQ_ERR_INVALID_ARGUMENT;
    LinearPlan p;
    int st = plan_linear(c, path, p);
    if (st != SWQ_OK) return st;
    if (dst_bytes < p.total) return SWQ_ERR_INVALID_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(dst) % 256 != 0) return SWQ_ERR_MISALIGNED;
    // shape: codes [.., rows, in*bits/32]; scales/biases [.., rows, in/group]
    const int64_t cols = p.w->shape.back();
    const int64_t rows_all = elements(std::vector<int64_t>(p.w->shape.begin(), p.w->shape.end() - 1));
    const int64_t in_dim = cols * (32 / p.bits);
    if (p.group <= 0 || in_dim % p.group != 0 || in_dim > INT32_MAX) return SWQ_ERR_BAD_SHAPE;
    const int64_t groups = in_dim / p.group;
    if (p.s->nbytes != rows_all * groups * scale_bytes(p.stype) || p.b->nbytes != p.s->nbytes)
        return SWQ_ERR_BAD_SHAPE;
    const int64_t rows = rows_per_expert > 0 ? rows_per_expert : rows_all;
    if (rows <= 0 || rows_all % rows != 0 || rows > INT32_MAX) return SWQ_ERR_BAD_SHAPE;
    uint8_t *d = static_cast<uint8_t *>(dst);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if ((st = c->staging.to_device(c->fds[p.w->file], p.w->begin, p.w->nbytes, d, s)) != SWQ_OK) return st;
    if ((st = c->staging.to_device(c->fds[p.s->file], p.s->begin, p.s->nbytes, d + p.s_off, s)) != SWQ_OK) return st;
    if ((st = c->staging.to_device(c->fds[p.b->file], p.b->begin, p.b->nbytes, d + p.b_off, s)) != SWQ_OK) return st;
    swq_qlinear q;
    std::memset(&q, 0, sizeof(q));
    q.w = q.scales = q.biases = dst;
    q.w_off = 0;
    q.s_off = p.s_off;
    q.b_off = p.b_off;
    q.out_dim = static_cast<int32_t>(rows);
    q.in_dim = static_cast<int32_t>(in_dim);
    q.group_size = p.group;
    q.bits = p.bits;
    q.scales_type = p.stype;
    if (rows_per_expert > 0) {  // ExpertStack strides (QwenMetalModel.swift:167-188)
        q.expert_stride_w = rows * cols * 4;
        q.expert_stride_sb = rows * groups * scale_bytes(p.stype);
    }
    *out = q;
    return SWQ_OK;
}

// ===========================================================================
// qpack

struct swq_qpack {
    struct Section {
        std::string name;
        Tensor t;  // dtype, per-expert shape; t.begin = offset inside the blob
    };
    std::string dir;
    int expert_count = 0, layer_count = 0;
    int64_t stride = 0;
    std::vector<Section> sections;
    std::vector<uint8_t> linear_layers;
    int quant_bits = 0, quant_group = 0;
    std::vector<int> fds;
    Staging staging;

    ~swq_qpack() {
        staging.release();
        for (int fd : fds)
            if (fd >= 0) close(fd);
    }

    const Section *section(const std::string &name) const {
        for (const auto &s : sections)
            if (s.name == name) return &s;
        return nullptr;
    }

    static bool get_int(const json::Value &o, const char *key, int64_t &v) {
        const json::Value *x = o.get(key);
        if (!x || !x->is_int()) return false;
        v = x->i;
        return true;
    }

    int open_dir(const std::string &d) {
        dir = d;
        std::string text;
        json::Value lay;
        if (!read_text(dir + "/packed_experts/layout.json", text)) return SWQ_ERR_IO;
        if (!json::parse(text, lay) || lay.kind != json::Value::Object) return SWQ_ERR_FORMAT;
        int64_t ec, lc;
        if (!get_int(lay, "expertCount", ec) || !get_int(lay, "layerCount", lc) ||
            !get_int(lay, "expertStride", stride))
            return SWQ_ERR_FORMAT;
        if (ec <= 0 || lc <= 0 || ec > (1 << 20) || lc > (1 << 16) || stride <= 0 || stride % kQpackPageAlignment != 0)
            return SWQ_ERR_FORMAT;
        expert_count = static_cast<int>(ec);
        layer_count = static_cast<int>(lc);
        const json::Value *secs = lay.get("sections");
        if (!secs || secs->kind != json::Value::Array) return SWQ_ERR_FORMAT;
        for (const auto &s : secs->arr) {
            Section sec;
            const json::Value *nm = s.get("name"), *dt = s.get("dtype");
            int64_t off, size;
            if (!nm || nm->kind != json::Value::String || !dt || dt->kind != json::Value::String ||
                !json_shape(s.get("shape"), sec.t.shape) || !get_int(s, "offset", off) || !get_int(s, "size", size))
                return SWQ_ERR_FORMAT;
            const int64_t es = dtype_size(dt->s), ne = elements(sec.t.shape);
            if (es == 0 || ne < 0 || ne * es != size || off < 0 || off + size > stride) return SWQ_ERR_FORMAT;
            sec.name = nm->s;
            sec.t.dtype = dt->s;
            sec.t.begin = off;
            sec.t.nbytes = size;
            sections.push_back(sec);
        }
        const json::Value *ll = lay.get("linearLayers");
        if (ll && ll->kind == json::Value::Array)
            for (const auto &b : ll->arr) linear_layers.push_back(b.kind == json::Value::Bool && b.b ? 1 : 0);
        // Manifest (Qpack.swift:37-46): quantBits / quantGroupSize, read by
        // QwenMetalModel (:137-152); optional here, needed by expert_linear.
        if (read_text(dir + "/manifest.json", text)) {
            json::Value man;
            if (!json::parse(text, man) || man.kind != json::Value::Object) return SWQ_ERR_FORMAT;
            const json::Value *magic = man.get("magic");
            int64_t version = 0, v;
            if (!magic || magic->kind != json::Value::String || magic->s != "QPACK" || !get_int(man, "version", version) ||
                version != 1)
                return SWQ_ERR_FORMAT;
            if (get_int(man, "quantBits", v)) quant_bits = static_cast<int>(v);
            if (get_int(man, "quantGroupSize", v)) quant_group = static_cast<int>(v);
        }
        fds.assign(static_cast<size_t>(layer_count), -1);
        return SWQ_OK;
    }

    // layer_NN.bin, opened on first use (QpackExpertReader.readExpert,
    // Qpack.swift:185-197); its size must be expertCount * expertStride.
    int layer_fd(int layer, int &fd) {
        if (layer < 0 || layer >= layer_count) return SWQ_ERR_INVALID_ARGUMENT;
        if (fds[layer] < 0) {
            char name[32];
            std::snprintf(name, sizeof(name), "layer_%02d.bin", layer);
            const int f = open((dir + "/packed_experts/" + name).c_str(), O_RDONLY | O_CLOEXEC);
            if (f < 0) return SWQ_ERR_IO;
            struct stat st;
            if (fstat(f, &st) != 0 || st.st_size != static_cast<int64_t>(expert_count) * stride) {
                close(f);
                return SWQ_ERR_FORMAT;
            }
            fds[layer] = f;
        }
        fd = fds[layer];
        return SWQ_OK;
    }
};

extern "C" int swq_qpack_open(const char *container_dir, swq_qpack **out) {
    if (!container_dir || !out) return SWQ_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    swq_qpack *q = new (std::nothrow) swq_qpack();
    if (!q) return SWQ_ERR_IO;
    int st;
    try {
        st = q->open_dir(container_dir);
    } catch (...) {
        st = SWQ_ERR_FORMAT;
    }
    if (st != SWQ_OK) {
        delete q;
        return st;
    }
    *out = q;
    return SWQ_OK;
}

extern "C" void swq_qpack_close(swq_qpack *q) { delete q; }

extern "C" int swq_qpack_layout(const swq_qpack *q, swq_qpack_layout_info *info) {
    if (!q || !info) return SWQ_ERR_INVALID_ARGUMENT;
    std::memset(info, 0, sizeof(*info));
    info->expert_count = q->expert_count;
    info->layer_count = q->layer_count;
    info->expert_stride = q->stride;
    info->quant_bits = q->quant_bits;
    info->quant_group_size = q->quant_group;
    info->section_count = static_cast<int32_t>(q->sections.size());
    return SWQ_OK;
}

extern "C" int swq_qpack_is_linear_layer(const swq_qpack *q, int layer) {
    if (!q || layer < 0 || layer >= static_cast<int>(q->linear_layers.size())) return SWQ_ERR_INVALID_ARGUMENT;
    return q->linear_layers[static_cast<size_t>(layer)];
}

extern "C" int swq_qpack_section(const swq_qpack *q, int index, const char **name, int64_t *offset,
                                 swq_tensor_info *info) {
    if (!q || index < 0 || index >= static_cast<int>(q->sections.size())) return SWQ_ERR_INVALID_ARGUMENT;
    const auto &s = q->sections[static_cast<size_t>(index)];
    if (name) *name = s.name.c_str();
    if (offset) *offset = s.t.begin;
    if (info) fill_info(s.t, info);
    return SWQ_OK;
}

extern "C" int swq_qpack_find_section(const swq_qpack *q, const char *name) {
    if (!q || !name) return SWQ_ERR_INVALID_ARGUMENT;
    for (size_t i = 0; i < q->sections.size(); ++i)
        if (q->sections[i].name == name) return static_cast<int>(i);
    return SWQ_ERR_MISSING_TENSOR;
}

extern "C" int swq_qpack_read_expert(swq_qpack *q, int layer, int expert, void *dst, int64_t dst_bytes) {
    if (!q || !dst || expert < 0 || expert >= (q ? q->expert_count : 0)) return SWQ_ERR_INVALID_ARGUMENT;
    if (dst_bytes < q->stride) return SWQ_ERR_INVALID_ARGUMENT;
    int fd, st;
    if ((st = q->layer_fd(layer, fd)) != SWQ_OK) return st;
    return read_exact(fd, dst, q->stride, static_cast<int64_t>(expert) * q->stride) ? SWQ_OK : SWQ_ERR_IO;
}

extern "C" int swq_qpack_load_experts(swq_qpack *q, int layer, int first_expert, int count, void *dst,
                                      int64_t dst_bytes, void *stream) {
    if (!q || !dst || first_expert < 0 || count <= 0 || first_expert > q->expert_count - count)
        return SWQ_ERR_INVALID_ARGUMENT;
    const int64_t n = static_cast<int64_t>(count) * q->stride;
    if (dst_bytes < n) return SWQ_ERR_INVALID_ARGUMENT;
    int fd, st;
    if ((st = q->layer_fd(layer, fd)) != SWQ_OK) return st;
    return q->staging.to_device(fd, static_cast<int64_t>(first_expert) * q->stride, n, static_cast<uint8_t *>(dst),
                                static_cast<hipStream_t>(stream));
}

extern "C" int swq_qpack_expert_linear(const swq_qpack *q, const void *base, const char *proj, swq_qlinear *out) {
    if (!q || !base || !proj || !out) return SWQ_ERR_INVALID_ARGUMENT;
    const std::string p(proj);
    const auto *w = q->section(p + ".weight");
    const auto *s = q->section(p + ".scales");
    const auto *b = q->section(p + ".biases");
    if (!w) return SWQ_ERR_MISSING_TENSOR;
    if (w->t.dtype != "U32") return SWQ_ERR_UNSUPPORTED_BITS;  // plain expert weights: not this kernel family
    if (!s || !b) return SWQ_ERR_MISSING_TENSOR;
    if (q->quant_bits == 0 || q->quant_group <= 0) return SWQ_ERR_FORMAT;
    if (q->quant_bits != 2 && q->quant_bits != 4 && q->quant_bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
    const int stype = scales_type_of(s->t.dtype);
    if (stype < 0 || b->t.dtype != s->t.dtype) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (w->t.shape.size() < 1) return SWQ_ERR_FORMAT;
    const int64_t cols = w->t.shape.back();
    const int64_t rows = elements(std::vector<int64_t>(w->t.shape.begin(), w->t.shape.end() - 1));
    const int64_t in_dim = cols * (32 / q->quant_bits);
    if (in_dim % q->quant_group != 0 || rows <= 0 || rows > INT32_MAX || in_dim > INT32_MAX) return SWQ_ERR_BAD_SHAPE;
    if (s->t.nbytes != rows * (in_dim / q->quant_group) * scale_bytes(stype) || b->t.nbytes != s->t.nbytes)
        return SWQ_ERR_BAD_SHAPE;
    swq_qlinear l;
    std::memset(&l, 0, sizeof(l));
    l.w = l.scales = l.biases = base;
    l.w_off = w->t.begin;
    l.s_off = s->t.begin;
    l.b_off = b->t.begin;
    l.out_dim = static_cast<int32_t>(rows);
    l.in_dim = static_cast<int32_t>(in_dim);
    l.group_size = q->quant_group;
    l.bits = q->quant_bits;
    l.scales_type = stype;
    l.expert_stride_w = q->stride;
    l.expert_stride_sb = q->stride;
    *out = l;
    return SWQ_OK;
}
