// iq_gguf.cpp -- GGUF checkpoint reader and expert residency loader
// (GgufCheckpoint, src/gguf.rs:1200-1460; warm_all_experts,
// src/residency.rs:39-131), behind the C ABI (include/iq_qgemm.h).
//
// The file is parsed on the host (GGUF v2/v3, little endian: magic, version,
// tensor and metadata counts, metadata key/values, tensor infos, then the
// tensor data at the next multiple of general.alignment).  Every read is
// bounds-checked against the file size, so a truncated or corrupt file is an
// error, never an out-of-range access.  Tensor bytes move to HBM through two
// pinned staging buffers: the read of one chunk overlaps the copy of the
// previous one.
#include <errno.h>
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/iq_qgemm.h"
#include "iq_api_internal.h"

#define IQ_API extern "C" __attribute__((visibility("default")))

namespace {

using namespace iq;

struct TensorInfo {
    std::string name;
    int dtype = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};  // GGUF order: ne[0] = columns (innermost)
    uint64_t offset = 0;           // absolute file offset of the first byte
    uint64_t nbytes = 0;           // 0 when the dtype's block size is unknown here
};

struct MetaValue {
    int type = -1;
    int64_t i = 0;
    double f = 0;
    std::string s;
};

// GGML type sizes (block elements, block bytes) of the types a checkpoint
// of this path holds; others are listed but cannot be loaded.
bool type_block(int t, int64_t* elems, int64_t* bytes) {
    switch (t) {
    case 0: *elems = 1; *bytes = 4; return true;      // F32
    case 1: *elems = 1; *bytes = 2; return true;      // F16
    case 30: *elems = 1; *bytes = 2; return true;     // BF16
    case 8: *elems = 32; *bytes = 34; return true;    // Q8_0
    case 12: *elems = 256; *bytes = 144; return true; // Q4_K
    case 13: *elems = 256; *bytes = 176; return true; // Q5_K
    case 14: *elems = 256; *bytes = 210; return true; // Q6_K
    default: return false;
    }
}

class Reader {
  public:
    Reader(int fd, uint64_t size) : fd_(fd), size_(size) {}
    uint64_t pos() const { return pos_; }
    bool read(void* dst, uint64_t n) {
        if (n > size_ || pos_ > size_ - n) return false;
        uint8_t* p = (uint8_t*)dst;
        uint64_t done = 0;
        while (done < n) {
            ssize_t r = pread(fd_, p + done, (size_t)std::min<uint64_t>(n - done, 1u << 30), (off_t)(pos_ + done));
            if (r <= 0) {
                if (r < 0 && errno == EINTR) continue;
                return false;
            }
            done += (uint64_t)r;
        }
        pos_ += n;
        return true;
    }
    template <class T>
    bool get(T* v) { return read(v, sizeof(T)); }
    bool str(std::string* s) {
        uint64_t n;
        if (!get(&n) || n > (1u << 24)) return false;  // keys and values are short
        s->resize(n);
        return n == 0 || read(&(*s)[0], n);
    }
    bool skip(uint64_t n) {
        if (n > size_ || pos_ > size_ - n) return false;
        pos_ += n;
        return true;
    }

  private:
    int fd_;
    uint64_t size_, pos_ = 0;
};

// Byte size of one scalar of a GGUF metadata type (0 for string/array).
int scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

bool read_scalar(Reader& r, uint32_t t, MetaValue* v) {
    v->type = (int)t;
    switch (t) {
    case 0: { uint8_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 1: { int8_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 2: { uint16_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 3: { int16_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 4: { uint32_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 5: { int32_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 6: { float x; if (!r.get(&x)) return false; v->f = x; v->i = (int64_t)x; return true; }
    case 7: { uint8_t x; if (!r.get(&x)) return false; v->i = x != 0; return true; }
    case 10: { uint64_t x; if (!r.get(&x)) return false; v->i = (int64_t)x; return true; }
    case 11: { int64_t x; if (!r.get(&x)) return false; v->i = x; return true; }
    case 12: { double x; if (!r.get(&x)) return false; v->f = x; v->i = (int64_t)x; return true; }
    case 8: return r.str(&v->s);
    default: return false;
    }
}

}  // namespace

struct iq_gguf {
    int fd = -1;
    std::string path;
    uint64_t file_size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::unordered_map<std::string, MetaValue> meta;
};

struct iq_experts {
    struct Layer {
        uint8_t* dev = nullptr;  // gate, up, down of one layer, each 256-byte aligned
        size_t gate_off = 0, up_off = 0, down_off = 0;
        size_t gate_bytes = 0, down_bytes = 0;
        int gate_dtype = 0, down_dtype = 0;
        int64_t n_experts = 0, inter = 0, hidden = 0;
    };
    std::vector<Layer> layers;
    size_t bytes = 0;
};

namespace {

int parse(iq_gguf* g) {
    Reader r(g->fd, g->file_size);
    uint32_t magic;
    if (!r.get(&magic)) return fail(IQ_ERR_SHAPE, "%s is too short to be a GGUF file", g->path.c_str());
    if (magic != 0x46554747u) return fail(IQ_ERR_SHAPE, "%s is not a GGUF file (bad magic)", g->path.c_str());
    if (!r.get(&g->version)) return fail(IQ_ERR_SHAPE, "truncated GGUF header");
    if (g->version < 2 || g->version > 3)
        return fail(IQ_ERR_SHAPE, "unsupported GGUF version %u (this reader takes versions 2 and 3)", g->version);
    uint64_t n_tensors, n_kv;
    if (!r.get(&n_tensors) || !r.get(&n_kv)) return fail(IQ_ERR_SHAPE, "truncated GGUF header");
    if (n_tensors > (1u << 24) || n_kv > (1u << 24)) return fail(IQ_ERR_SHAPE, "implausible GGUF counts");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        uint32_t t;
        if (!r.str(&key) || !r.get(&t)) return fail(IQ_ERR_SHAPE, "truncated GGUF metadata (entry %llu)",
                                                      (unsigned long long)i);
        MetaValue v;
        if (t == 9) {  // array: element type, count, elements (kept as a count only)
            uint32_t et;
            uint64_t cnt;
            if (!r.get(&et) || !r.get(&cnt)) return fail(IQ_ERR_SHAPE, "truncated GGUF array %s", key.c_str());
            v.type = 9;
            v.i = (int64_t)cnt;
            if (et == 8) {
                for (uint64_t j = 0; j < cnt; j++) {
                    std::string s;
                    if (!r.str(&s)) return fail(IQ_ERR_SHAPE, "truncated GGUF string array %s", key.c_str());
                }
            } else {
                const int sz = scalar_size(et);
                if (!sz || cnt > (uint64_t)1 << 40 || !r.skip(cnt * (uint64_t)sz))
                    return fail(IQ_ERR_SHAPE, "bad GGUF array %s (type %u)", key.c_str(), et);
            }
        } else if (!read_scalar(r, t, &v)) {
            return fail(IQ_ERR_SHAPE, "bad GGUF metadata value %s (type %u)", key.c_str(), t);
        }
        g->meta[key] = v;
    }
    auto al = g->meta.find("general.alignment");
    if (al != g->meta.end()) {
        if (al->second.i <= 0 || (al->second.i & (al->second.i - 1)))
            return fail(IQ_ERR_SHAPE, "GGUF alignment %lld is not a power of two", (long long)al->second.i);
        g->alignment = (uint64_t)al->second.i;
    }
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        TensorInfo& ti = g->tensors[i];
        uint32_t nd, t;
        if (!r.str(&ti.name) || !r.get(&nd)) return fail(IQ_ERR_SHAPE, "truncated GGUF tensor info %llu",
                                                         (unsigned long long)i);
        if (nd < 1 || nd > 4) return fail(IQ_ERR_SHAPE, "GGUF tensor %s has %u dimensions", ti.name.c_str(), nd);
        ti.n_dims = (int)nd;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t ne;
            if (!r.get(&ne)) return fail(IQ_ERR_SHAPE, "truncated GGUF tensor info %s", ti.name.c_str());
            if (ne == 0 || ne > ((uint64_t)1 << 40)) return fail(IQ_ERR_SHAPE, "bad GGUF dimension in %s", ti.name.c_str());
            ti.ne[d] = (int64_t)ne;
        }
        uint64_t off;
        if (!r.get(&t) || !r.get(&off)) return fail(IQ_ERR_SHAPE, "truncated GGUF tensor info %s", ti.name.c_str());
        ti.dtype = (int)t;
        ti.offset = off;  // relative until the data start is known
        int64_t be, bb;
        if (type_block(ti.dtype, &be, &bb)) {
            if (ti.ne[0] % be) return fail(IQ_ERR_SHAPE, "GGUF tensor %s width %lld is not a whole number of blocks",
                                           ti.name.c_str(), (long long)ti.ne[0]);
            uint64_t n = (uint64_t)(ti.ne[0] / be) * (uint64_t)bb;
            for (int d = 1; d < ti.n_dims; d++)
                if (__builtin_mul_overflow(n, (uint64_t)ti.ne[d], &n))
                    return fail(IQ_ERR_SHAPE, "GGUF tensor %s byte size overflows", ti.name.c_str());
            ti.nbytes = n;
        }
        if (!g->by_name.emplace(ti.name, i).second)
            return fail(IQ_ERR_SHAPE, "GGUF tensor %s appears twice", ti.name.c_str());
    }
    g->data_offset = (r.pos() + g->alignment - 1) / g->alignment * g->alignment;
    for (TensorInfo& ti : g->tensors) {
        if (ti.offset % g->alignment)
            return fail(IQ_ERR_SHAPE, "GGUF tensor %s is not aligned to %llu bytes", ti.name.c_str(),
                        (unsigned long long)g->alignment);
        if (__builtin_add_overflow(ti.offset, g->data_offset, &ti.offset))
            return fail(IQ_ERR_SHAPE, "GGUF tensor %s offset overflows", ti.name.c_str());
        if (ti.offset > g->file_size || ti.nbytes > g->file_size - ti.offset)
            return fail(IQ_ERR_SHAPE, "GGUF tensor %s extends past the end of the file", ti.name.c_str());
    }
    return IQ_OK;
}

const TensorInfo* find(const iq_gguf* g, const char* name) {
    if (!name) return nullptr;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

// Copy file bytes [off, off + n) to device memory through two pinned
// staging buffers on `s` (the read of one chunk overlaps the copy of the
// previous one).  Synchronises before returning.
int upload_range(const iq_gguf* g, uint64_t off, uint64_t n, uint8_t* dev, hipStream_t s) {
    constexpr size_t kChunk = (size_t)32 << 20;
    uint8_t* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = IQ_OK;
    for (int i = 0; i < 2 && rc == IQ_OK; i++) {
        if (hipHostMalloc((void**)&stage[i], kChunk, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            rc = fail(IQ_ERR_OOM, "pinned staging buffer of %zu bytes", kChunk);
        } else if (hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) {
            rc = fail(IQ_ERR_HIP, "hipEventCreate");
        }
    }
    uint64_t pos = 0;
    for (int k = 0; rc == IQ_OK && pos < n; k ^= 1) {
        const size_t len = (size_t)std::min<uint64_t>(kChunk, n - pos);
        if (hipEventSynchronize(done[k]) != hipSuccess) {  // the copy that last used this buffer
            rc = fail(IQ_ERR_HIP, "hipEventSynchronize");
            break;
        }
        Reader r(g->fd, g->file_size);
        if (!r.skip(off + pos) || !r.read(stage[k], len)) {
            rc = fail(IQ_ERR_SHAPE, "short read of %s at offset %llu", g->path.c_str(), (unsigned long long)(off + pos));
            break;
        }
        hipError_t e = hipMemcpyAsync(dev + pos, stage[k], len, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(done[k], s);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync (GGUF upload)");
        pos += len;
    }
    if (hipStreamSynchronize(s) != hipSuccess && rc == IQ_OK) rc = fail(IQ_ERR_HIP, "hipStreamSynchronize");
    for (int i = 0; i < 2; i++) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    return rc;
}

const char* type_name(int t) {
    switch (t) {
    case 0: return "F32";
    case 1: return "F16";
    case 30: return "BF16";
    case 8: return "Q8_0";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    default: return "unsupported";
    }
}

}  // namespace

IQ_API int iq_gguf_open(const char* path, iq_gguf_t* out) {
    if (!path || !out) return fail(IQ_ERR_INVALID, "null pointer");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(IQ_ERR_INVALID, "cannot open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(IQ_ERR_INVALID, "cannot stat %s: %s", path, strerror(errno));
    }
    iq_gguf* g = new iq_gguf;
    g->fd = fd;
    g->path = path;
    g->file_size = (uint64_t)st.st_size;
    if (int rc = parse(g)) {
        close(fd);
        delete g;
        return rc;
    }
    *out = g;
    return IQ_OK;
}

IQ_API int iq_gguf_close(iq_gguf_t g) {
    if (!g) return IQ_OK;
    if (g->fd >= 0) close(g->fd);
    delete g;
    return IQ_OK;
}

IQ_API int64_t iq_gguf_tensor_count(iq_gguf_t g) { return g ? (int64_t)g->tensors.size() : -1; }

IQ_API const char* iq_gguf_tensor_name(iq_gguf_t g, int64_t index) {
    if (!g || index < 0 || index >= (int64_t)g->tensors.size()) return nullptr;
    return g->tensors[(size_t)index].name.c_str();
}

IQ_API int iq_gguf_tensor_info(iq_gguf_t g, const char* name, int* dtype, int* n_dims, int64_t dims[4],
                               uint64_t* file_offset, uint64_t* nbytes) {
    if (!g) return fail(IQ_ERR_INVALID, "null GGUF handle");
    const TensorInfo* ti = find(g, name);
    if (!ti) return fail(IQ_ERR_RANGE, "GGUF is missing tensor \"%s\"", name ? name : "(null)");
    if (dtype) *dtype = ti->dtype;
    if (n_dims) *n_dims = ti->n_dims;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = d < ti->n_dims ? ti->ne[ti->n_dims - 1 - d] : 0;
    if (file_offset) *file_offset = ti->offset;
    if (nbytes) *nbytes = ti->nbytes;
    return IQ_OK;
}

IQ_API int iq_gguf_meta_int(iq_gguf_t g, const char* key, int64_t* value) {
    if (!g || !key || !value) return fail(IQ_ERR_INVALID, "null pointer");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return fail(IQ_ERR_RANGE, "GGUF has no metadata key \"%s\"", key);
    if (it->second.type == 8) return fail(IQ_ERR_DTYPE, "GGUF metadata \"%s\" is a string", key);
    *value = it->second.i;
    return IQ_OK;
}

IQ_API const char* iq_gguf_meta_str(iq_gguf_t g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() || it->second.type != 8 ? nullptr : it->second.s.c_str();
}

IQ_API int iq_gguf_load_matrix(iq_gguf_t g, const char* name, iq_weight_t* out) {
    if (!g || !out) return fail(IQ_ERR_INVALID, "null pointer");
    const TensorInfo* ti = find(g, name);
    if (!ti) return fail(IQ_ERR_RANGE, "GGUF is missing tensor \"%s\"", name ? name : "(null)");
    if (ti->n_dims != 2)
        return fail(IQ_ERR_SHAPE, "GGUF tensor \"%s\" has %d dimensions, expected a matrix", name, ti->n_dims);
    if (!dtype_ok(ti->dtype))
        return fail(IQ_ERR_DTYPE, "unsupported executable GGUF matrix dtype %s for \"%s\"", type_name(ti->dtype), name);
    iq_weight_t w = nullptr;
    // the upload path's shape checks and allocation, then stream the bytes
    int64_t rb;
    if (int rc = check_matrix(ti->dtype, ti->ne[1], ti->ne[0], (size_t)ti->nbytes, &rb)) return rc;
    if (int rc = alloc_weight(ti->dtype, ti->ne[1], ti->ne[0], rb, &w)) return rc;
    if (int rc = upload_range(g, ti->offset, ti->nbytes, w->dev, nullptr)) {
        iq_weights_free(w);
        return rc;
    }
    *out = w;
    return IQ_OK;
}

IQ_API int iq_gguf_upload_tensor(iq_gguf_t g, const char* name, void* device_dst, size_t capacity,
                                 iq_stream_t stream) {
    if (!g || !device_dst) return fail(IQ_ERR_INVALID, "null pointer");
    const TensorInfo* ti = find(g, name);
    if (!ti) return fail(IQ_ERR_RANGE, "GGUF is missing tensor \"%s\"", name ? name : "(null)");
    if (!ti->nbytes) return fail(IQ_ERR_DTYPE, "GGUF tensor \"%s\" has dtype %d, which this reader cannot size", name,
                                 ti->dtype);
    if (capacity < ti->nbytes)
        return fail(IQ_ERR_SHAPE, "GGUF tensor \"%s\" has %llu bytes; the buffer holds %zu", name,
                    (unsigned long long)ti->nbytes, capacity);
    return upload_range(g, ti->offset, ti->nbytes, (uint8_t*)device_dst, (hipStream_t)stream);
}

IQ_API int iq_gguf_load_experts(iq_gguf_t g, int64_t n_layers, iq_experts_t* out) {
    if (!g || !out) return fail(IQ_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (n_layers <= 0) return fail(IQ_ERR_SHAPE, "invalid layer count %lld", (long long)n_layers);
    static const char* kSuffix[3] = {"ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"};
    struct Item {
        const TensorInfo* ti;
        int64_t layer;
        int part;
    };
    std::vector<Item> items;
    iq_experts* R = new iq_experts;
    R->layers.resize((size_t)n_layers);
    for (int64_t l = 0; l < n_layers; l++) {
        const TensorInfo* t[3];
        for (int p = 0; p < 3; p++) {
            const std::string name = "blk." + std::to_string(l) + "." + kSuffix[p];
            t[p] = find(g, name.c_str());
            if (!t[p]) {
                delete R;
                return fail(IQ_ERR_RANGE, "GGUF is missing expert tensor \"%s\"", name.c_str());
            }
            if (t[p]->n_dims != 3) {
                delete R;
                return fail(IQ_ERR_SHAPE, "GGUF tensor \"%s\" has %d dimensions, expected [experts, rows, columns]",
                            name.c_str(), t[p]->n_dims);
            }
            if (!moe_dtype_ok(t[p]->dtype)) {
                delete R;
                return fail(IQ_ERR_DTYPE, "unsupported expert dtype %s for \"%s\"", type_name(t[p]->dtype),
                            name.c_str());
            }
            items.push_back(Item{t[p], l, p});
        }
        // gate and up pair into one product: same dtype and shape (GgufExpertPair, src/gguf.rs:1321-1360)
        if (t[0]->dtype != t[1]->dtype || t[0]->ne[0] != t[1]->ne[0] || t[0]->ne[1] != t[1]->ne[1] ||
            t[0]->ne[2] != t[1]->ne[2]) {
            delete R;
            return fail(IQ_ERR_SHAPE, "cannot pair expert tensors blk.%lld gate and up with different dtypes or shapes",
                        (long long)l);
        }
        // down is [experts, hidden, inter] against gate's [experts, inter, hidden]
        if (t[2]->ne[2] != t[0]->ne[2] || t[2]->ne[0] != t[0]->ne[1] || t[2]->ne[1] != t[0]->ne[0]) {
            delete R;
            return fail(IQ_ERR_SHAPE, "blk.%lld down experts do not match gate/up", (long long)l);
        }
        iq_experts::Layer& L = R->layers[(size_t)l];
        L.gate_dtype = t[0]->dtype;
        L.down_dtype = t[2]->dtype;
        L.n_experts = t[0]->ne[2];
        L.inter = t[0]->ne[1];
        L.hidden = t[0]->ne[0];
        L.gate_bytes = (size_t)t[0]->nbytes;
        L.down_bytes = (size_t)t[2]->nbytes;
        auto a256 = [](size_t v) { return (v + 255) & ~(size_t)255; };
        L.gate_off = 0;
        L.up_off = a256(L.gate_bytes);
        L.down_off = L.up_off + a256(L.gate_bytes);
        const size_t total = L.down_off + a256(L.down_bytes) + 256;  // padding past the last block
        if (hipMalloc(&L.dev, total) != hipSuccess) {
            (void)hipGetLastError();
            iq_experts_free(R);
            return fail(IQ_ERR_OOM, "expert residency of layer %lld (%zu bytes) does not fit", (long long)l, total);
        }
        if (hipMemset(L.dev, 0, total) != hipSuccess) {
            iq_experts_free(R);
            return fail(IQ_ERR_HIP, "hipMemset (expert residency)");
        }
    }
    // file order keeps the reads sequential (warm_all_experts sorts by offset)
    std::sort(items.begin(), items.end(), [](const Item& a, const Item& b) { return a.ti->offset < b.ti->offset; });
    hipStream_t s;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        iq_experts_free(R);
        return fail(IQ_ERR_HIP, "hipStreamCreate");
    }
    for (const Item& it : items) {
        iq_experts::Layer& L = R->layers[(size_t)it.layer];
        const size_t off = it.part == 0 ? L.gate_off : it.part == 1 ? L.up_off : L.down_off;
        if (int rc = upload_range(g, it.ti->offset, it.ti->nbytes, L.dev + off, s)) {
            (void)hipStreamDestroy(s);
            iq_experts_free(R);
            return rc;
        }
        R->bytes += (size_t)it.ti->nbytes;
    }
    (void)hipStreamDestroy(s);
    *out = R;
    return IQ_OK;
}

IQ_API int iq_experts_free(iq_experts_t r) {
    if (!r) return IQ_OK;
    for (auto& L : r->layers)
        if (L.dev) (void)hipFree(L.dev);
    delete r;
    return IQ_OK;
}

IQ_API size_t iq_experts_bytes(iq_experts_t r) { return r ? r->bytes : 0; }

IQ_API int iq_experts_layer(iq_experts_t r, int64_t layer, iq_moe_desc* desc) {
    if (!r || !desc) return fail(IQ_ERR_INVALID, "null pointer");
    if (layer < 0 || layer >= (int64_t)r->layers.size())
        return fail(IQ_ERR_RANGE, "layer %lld out of range (%zu resident layers)", (long long)layer, r->layers.size());
    const iq_experts::Layer& L = r->layers[(size_t)layer];
    desc->hidden = L.hidden;
    desc->inter = L.inter;
    desc->n_experts = L.n_experts;
    desc->gate_dtype = L.gate_dtype;
    desc->down_dtype = L.down_dtype;
    desc->gate = L.dev + L.gate_off;
    desc->up = L.dev + L.up_off;
    desc->down = L.dev + L.down_off;
    desc->gate_bytes = L.gate_bytes;
    desc->up_bytes = L.gate_bytes;
    desc->down_bytes = L.down_bytes;
    return IQ_OK;
}
