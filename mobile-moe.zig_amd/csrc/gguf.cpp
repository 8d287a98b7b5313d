// GGUF v3 container (gguf.zig:266-413) and weight binding (model.zig:236-395)
// for device-resident weights: the file is memory-mapped once, its header,
// metadata and tensor descriptors are parsed from the mapping, and tensors
// are uploaded to the device once, into the tile layout the kernels read.
//
// Parsing works on the mapped bytes through a cursor that checks every read
// against the file size (the reference reads the header with read(2) and
// maps afterwards; the parsed result is the same). Limits and failures follow
// parse / readString / readMetadataValue (gguf.zig:266-363, 444-555): magic
// "GGUF", version 3, strings of at most 65,536 bytes, arrays of at most 10^7
// elements, at most 4 dimensions, alignment from general.alignment (u32 or
// u64) else 32, tensor data at the first aligned offset after the tensor
// descriptors. Metadata values and tensor descriptors with a repeated key
// replace the earlier one, keeping its position (StringArrayHashMap.put).
#include <errno.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mmhip.h"
#include "backend.hpp"

using mmhip::set_error;

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF", little-endian
constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMaxString = 65536;
constexpr uint64_t kMaxArray = 10000000;

enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

int scalar_size(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

struct Value {
    uint32_t type = 0;
    uint64_t bits = 0;          // scalar: the little-endian bytes, zero-extended
    const uint8_t* ptr = nullptr;  // string bytes / array payload in the mapping
    uint64_t len = 0;           // string bytes / array elements
    uint64_t nbytes = 0;        // array payload bytes
    uint32_t elem = 0;          // array element type
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
};

struct ParseError {
    int code;
    std::string what;
};

struct Cursor {
    const uint8_t* base;
    uint64_t size, pos = 0;

    const uint8_t* take(uint64_t n) {
        if (n > size - pos) throw ParseError{MMHIP_ERR_INVALID, "EndOfStream at byte " + std::to_string(pos)};
        const uint8_t* p = base + pos;
        pos += n;
        return p;
    }
    uint64_t uint(int bytes) {
        const uint8_t* p = take(bytes);
        uint64_t v = 0;
        for (int i = bytes - 1; i >= 0; --i) v = (v << 8) | p[i];
        return v;
    }
    uint32_t u32() { return (uint32_t)uint(4); }
    uint64_t u64() { return uint(8); }
    std::pair<const uint8_t*, uint64_t> str() {
        const uint64_t n = u64();
        if (n > kMaxString) throw ParseError{MMHIP_ERR_INVALID, "StringTooLong (" + std::to_string(n) + " bytes)"};
        return {take(n), n};
    }
};

Value read_value(Cursor& c, uint32_t type) {
    Value v;
    v.type = type;
    if (const int sz = scalar_size(type)) {
        v.bits = c.uint(sz);
        return v;
    }
    if (type == kString) {
        auto s = c.str();
        v.ptr = s.first;
        v.len = s.second;
        return v;
    }
    if (type != kArray) throw ParseError{MMHIP_ERR_UNSUPPORTED, "UnsupportedMetadataType " + std::to_string(type)};
    v.elem = c.u32();
    v.len = c.u64();
    if (v.len > kMaxArray) throw ParseError{MMHIP_ERR_INVALID, "ArrayTooLong (" + std::to_string(v.len) + ")"};
    const uint64_t start = c.pos;
    if (v.elem == kString) {
        for (uint64_t i = 0; i < v.len; ++i) c.str();
    } else if (const int sz = scalar_size(v.elem)) {
        c.take(v.len * (uint64_t)sz);
    } else {
        throw ParseError{MMHIP_ERR_UNSUPPORTED, "UnsupportedArrayType " + std::to_string(v.elem)};
    }
    v.ptr = c.base + start;
    v.nbytes = c.pos - start;
    return v;
}

uint64_t block_elems(uint32_t t) { return t == MMHIP_TYPE_Q8_0 ? 32 : t == MMHIP_TYPE_IQ2_XXS ? 256 : 1; }
uint64_t block_bytes(uint32_t t) {
    switch (t) {
        case MMHIP_TYPE_F32: return 4;
        case MMHIP_TYPE_F16: return 2;
        case MMHIP_TYPE_Q8_0: return 34;
        case MMHIP_TYPE_IQ2_XXS: return 66;
        default: return 0;
    }
}

}  // namespace

struct mmhip_gguf {
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t tensor_count = 0, metadata_count = 0;
    uint64_t alignment = kDefaultAlignment, data_offset = 0;
    std::vector<std::string> keys;                 // first-occurrence order
    std::unordered_map<std::string, Value> meta;
    std::vector<Tensor> tensors;                   // first-occurrence order
    std::unordered_map<std::string, size_t> tensor_index;

    ~mmhip_gguf() {
        if (map) munmap(const_cast<uint8_t*>(map), size);
    }
};

namespace {

void parse(mmhip_gguf& g) {
    Cursor c{g.map, g.size};
    if (c.u32() != kMagic) throw ParseError{MMHIP_ERR_INVALID, "InvalidMagic"};
    g.version = c.u32();
    if (g.version != kVersion) throw ParseError{MMHIP_ERR_INVALID, "UnsupportedVersion " + std::to_string(g.version)};
    g.tensor_count = c.u64();
    g.metadata_count = c.u64();
    for (uint64_t i = 0; i < g.metadata_count; ++i) {
        auto k = c.str();
        std::string key((const char*)k.first, k.second);
        const uint32_t type = c.u32();
        Value v = read_value(c, type);
        if (g.meta.find(key) == g.meta.end()) g.keys.push_back(key);
        g.meta[key] = v;
    }
    for (uint64_t i = 0; i < g.tensor_count; ++i) {
        Tensor t;
        auto n = c.str();
        t.name.assign((const char*)n.first, n.second);
        t.n_dims = c.u32();
        if (t.n_dims > 4) throw ParseError{MMHIP_ERR_INVALID, "TooManyDimensions (" + std::to_string(t.n_dims) + ")"};
        for (uint32_t d = 0; d < t.n_dims; ++d) t.dims[d] = c.u64();
        t.type = c.u32();
        t.offset = c.u64();
        auto it = g.tensor_index.find(t.name);
        if (it == g.tensor_index.end()) {
            g.tensor_index.emplace(t.name, g.tensors.size());
            g.tensors.push_back(t);
        } else {
            g.tensors[it->second] = t;
        }
    }
    auto al = g.meta.find("general.alignment");
    if (al != g.meta.end() && (al->second.type == kU32 || al->second.type == kU64)) g.alignment = al->second.bits;
    if (g.alignment == 0) throw ParseError{MMHIP_ERR_INVALID, "general.alignment is 0"};
    g.data_offset = c.pos + (g.alignment - c.pos % g.alignment) % g.alignment;
}

void describe(const mmhip_gguf& g, const Tensor& t, mmhip_gguf_tensor* out) {
    std::memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->dims[d] = t.dims[d];
    out->type = t.type;
    out->offset = t.offset;
    uint64_t n = 1;
    bool overflow = false;
    for (uint32_t d = 0; d < t.n_dims; ++d) overflow |= __builtin_mul_overflow(n, t.dims[d], &n);
    out->n_elements = overflow ? 0 : n;
    if (overflow) return;  // no byte count, no data pointer
    const uint64_t bb = block_bytes(t.type), be = block_elems(t.type);
    out->n_bytes = bb ? (n + be - 1) / be * bb : 0;
    // Data pointer only for a type this library reads whose bytes lie inside the file.
    const uint64_t start = g.data_offset + t.offset;
    if (bb && start >= g.data_offset && start <= g.size && out->n_bytes <= g.size - start)
        out->data = g.map + start;
}

const Value* lookup(const mmhip_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

int not_found(const std::string& what) {
    set_error(MMHIP_ERR_NOT_FOUND, what);
    return MMHIP_ERR_NOT_FOUND;
}

// A matrix stack from a tensor: ggml's dims[0] is the row length, dims[1]
// the rows, dims[2] the stacked matrices (ffn_*_exps: [cols, rows, experts]).
int tensor_matrix(const mmhip_gguf* g, const std::string& name, mmhip_gguf_tensor* t) {
    if (int rc = mmhip_gguf_find_tensor(g, name.c_str(), t)) return rc;
    if (!t->data) {
        set_error(MMHIP_ERR_INVALID, name + ": unsupported type " + std::to_string(t->type) +
                                         " or data outside the file");
        return MMHIP_ERR_INVALID;
    }
    if (t->dims[3] != 1 || t->n_elements == 0) {
        set_error(MMHIP_ERR_INVALID, name + ": not a stack of matrices");
        return MMHIP_ERR_INVALID;
    }
    // The upload reads whole blocks per row: rows must not share a block.
    if (t->dims[0] % block_elems(t->type) != 0) {
        set_error(MMHIP_ERR_INVALID, name + ": row length is not a whole number of blocks");
        return MMHIP_ERR_INVALID;
    }
    return MMHIP_OK;
}

}  // namespace

extern "C" {

int mmhip_gguf_open(const char* path, mmhip_gguf** out) {
    if (!path || !out) {
        set_error(MMHIP_ERR_INVALID, "gguf_open: null pointer");
        return MMHIP_ERR_INVALID;
    }
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        set_error(MMHIP_ERR_INVALID, std::string("gguf_open: cannot open ") + path + ": " + std::strerror(errno));
        return MMHIP_ERR_INVALID;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || st.st_size <= 0) {
        close(fd);
        set_error(MMHIP_ERR_INVALID, std::string("gguf_open: not a non-empty regular file: ") + path);
        return MMHIP_ERR_INVALID;
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        set_error(MMHIP_ERR_NOMEM, std::string("gguf_open: mmap: ") + std::strerror(errno));
        return MMHIP_ERR_NOMEM;
    }
    madvise(m, (size_t)st.st_size, MADV_WILLNEED);
    auto* g = new mmhip_gguf;
    g->map = static_cast<const uint8_t*>(m);
    g->size = (uint64_t)st.st_size;
    try {
        parse(*g);
    } catch (const ParseError& e) {
        delete g;
        set_error(e.code, "gguf_open: " + e.what);
        return e.code;
    }
    *out = g;
    return MMHIP_OK;
}

void mmhip_gguf_close(mmhip_gguf* g) { delete g; }

int mmhip_gguf_get_info(const mmhip_gguf* g, mmhip_gguf_info* out) {
    if (!g || !out) {
        set_error(MMHIP_ERR_INVALID, "gguf_get_info: null pointer");
        return MMHIP_ERR_INVALID;
    }
    out->version = g->version;
    out->tensor_count = g->tensor_count;
    out->metadata_count = g->metadata_count;
    out->n_tensors = g->tensors.size();
    out->n_keys = g->keys.size();
    out->alignment = g->alignment;
    out->data_offset = g->data_offset;
    out->file_size = g->size;
    return MMHIP_OK;
}

int mmhip_gguf_tensor_at(const mmhip_gguf* g, uint64_t index, mmhip_gguf_tensor* out) {
    if (!g || !out || index >= g->tensors.size()) {
        set_error(MMHIP_ERR_INVALID, "gguf_tensor_at: null pointer or index out of range");
        return MMHIP_ERR_INVALID;
    }
    describe(*g, g->tensors[index], out);
    return MMHIP_OK;
}

int mmhip_gguf_find_tensor(const mmhip_gguf* g, const char* name, mmhip_gguf_tensor* out) {
    if (!g || !name || !out) {
        set_error(MMHIP_ERR_INVALID, "gguf_find_tensor: null pointer");
        return MMHIP_ERR_INVALID;
    }
    auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return not_found(std::string("tensor ") + name + " not in the file");
    describe(*g, g->tensors[it->second], out);
    return MMHIP_OK;
}

const char* mmhip_gguf_key_at(const mmhip_gguf* g, uint64_t index) {
    return g && index < g->keys.size() ? g->keys[index].c_str() : nullptr;
}

int mmhip_gguf_meta_type(const mmhip_gguf* g, const char* key) {
    const Value* v = lookup(g, key);
    return v ? (int)v->type : not_found(std::string("metadata key ") + (key ? key : "(null)"));
}

int mmhip_gguf_meta_int(const mmhip_gguf* g, const char* key, int64_t* out) {
    const Value* v = lookup(g, key);
    if (!v || !out) return not_found(std::string("integer metadata ") + (key ? key : "(null)"));
    switch (v->type) {
        case kU8: case kU16: case kU32: *out = (int64_t)v->bits; return MMHIP_OK;
        case kI8: *out = (int8_t)v->bits; return MMHIP_OK;
        case kI16: *out = (int16_t)v->bits; return MMHIP_OK;
        case kI32: *out = (int32_t)v->bits; return MMHIP_OK;
        case kI64: *out = (int64_t)v->bits; return MMHIP_OK;
        case kU64:
            if (v->bits > (uint64_t)INT64_MAX) {
                set_error(MMHIP_ERR_INVALID, std::string(key) + ": u64 value does not fit i64");
                return MMHIP_ERR_INVALID;
            }
            *out = (int64_t)v->bits;
            return MMHIP_OK;
        default: return not_found(std::string(key) + " is not an integer");
    }
}

int mmhip_gguf_meta_float(const mmhip_gguf* g, const char* key, double* out) {
    const Value* v = lookup(g, key);
    if (!v || !out) return not_found(std::string("float metadata ") + (key ? key : "(null)"));
    if (v->type == kF32) {
        float f;
        const uint32_t b = (uint32_t)v->bits;
        std::memcpy(&f, &b, 4);
        *out = f;
        return MMHIP_OK;
    }
    if (v->type == kF64) {
        std::memcpy(out, &v->bits, 8);
        return MMHIP_OK;
    }
    return not_found(std::string(key) + " is not a float");
}

int mmhip_gguf_meta_string(const mmhip_gguf* g, const char* key, const char** str, uint64_t* len) {
    const Value* v = lookup(g, key);
    if (!v || !str || !len || v->type != kString) return not_found(std::string("string metadata ") + (key ? key : "(null)"));
    *str = (const char*)v->ptr;
    *len = v->len;
    return MMHIP_OK;
}

int mmhip_gguf_meta_array(const mmhip_gguf* g, const char* key, uint32_t* elem_type, uint64_t* len,
                          const void** data, uint64_t* n_bytes) {
    const Value* v = lookup(g, key);
    if (!v || !elem_type || !len || !data || !n_bytes || v->type != kArray)
        return not_found(std::string("array metadata ") + (key ? key : "(null)"));
    *elem_type = v->elem;
    *len = v->len;
    *data = v->ptr;
    *n_bytes = v->nbytes;
    return MMHIP_OK;
}

int mmhip_weight_upload_gguf(mmhip_ctx* ctx, const mmhip_gguf* g, const char* name, mmhip_weight** out_w) {
    if (!g || !name || !out_w) {
        set_error(MMHIP_ERR_INVALID, "weight_upload_gguf: null pointer");
        return MMHIP_ERR_INVALID;
    }
    mmhip_gguf_tensor t;
    if (int rc = tensor_matrix(g, name, &t)) return rc;
    return mmhip_weight_upload(ctx, t.data, t.type, t.dims[1], t.dims[0], t.dims[2], out_w);
}

int mmhip_weight_upload_gguf_rows(mmhip_ctx* ctx, const mmhip_gguf* g, const char* const* names, uint32_t n,
                                  mmhip_weight** out_w) {
    if (!g || !names || n == 0 || !out_w) {
        set_error(MMHIP_ERR_INVALID, "weight_upload_gguf_rows: null pointer or no tensors");
        return MMHIP_ERR_INVALID;
    }
    std::vector<mmhip_gguf_tensor> ts(n);
    uint64_t rows = 0, bytes = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (!names[i]) {
            set_error(MMHIP_ERR_INVALID, "weight_upload_gguf_rows: null tensor name");
            return MMHIP_ERR_INVALID;
        }
        if (int rc = tensor_matrix(g, names[i], &ts[i])) return rc;
        if (ts[i].dims[2] != 1 || ts[i].type != ts[0].type || ts[i].dims[0] != ts[0].dims[0]) {
            set_error(MMHIP_ERR_INVALID, std::string("weight_upload_gguf_rows: ") + names[i] +
                                             " is not one matrix of the first tensor's type and row length");
            return MMHIP_ERR_INVALID;
        }
        rows += ts[i].dims[1];
        bytes += ts[i].n_bytes;
    }
    // Rows of whole blocks are contiguous in GGUF, so the stacked matrix is
    // the tensors' bytes back to back; it is staged on the device once.
    void* staging = nullptr;
    if (int rc = mmhip_malloc(ctx, &staging, bytes)) return rc;
    int rc = MMHIP_OK;
    uint64_t off = 0;
    for (uint32_t i = 0; i < n && rc == MMHIP_OK; ++i) {
        rc = mmhip_memcpy_h2d(ctx, static_cast<char*>(staging) + off, ts[i].data, ts[i].n_bytes);
        off += ts[i].n_bytes;
    }
    // weight_from_device synchronises after its repack, so the staging copy
    // is free to release once it returns; on failure *out_w stays null.
    if (rc == MMHIP_OK) rc = mmhip_weight_from_device(ctx, staging, ts[0].type, rows, ts[0].dims[0], 1, out_w);
    mmhip_free(ctx, staging);
    return rc;
}

int mmhip_moe_layer_create_gguf(mmhip_ctx* ctx, const mmhip_gguf* g, uint32_t layer, mmhip_moe_layer** out_layer) {
    if (!g || !out_layer) {
        set_error(MMHIP_ERR_INVALID, "moe_layer_create_gguf: null pointer");
        return MMHIP_ERR_INVALID;
    }
    const std::string p = "blk." + std::to_string(layer) + ".";
    mmhip_gguf_tensor router, gate, up, down;
    if (int rc = tensor_matrix(g, p + "ffn_gate_inp.weight", &router)) return rc;
    if (int rc = tensor_matrix(g, p + "ffn_gate_exps.weight", &gate)) return rc;
    if (int rc = tensor_matrix(g, p + "ffn_up_exps.weight", &up)) return rc;
    if (int rc = tensor_matrix(g, p + "ffn_down_exps.weight", &down)) return rc;
    const uint64_t hidden = gate.dims[0], inter = gate.dims[1], experts = gate.dims[2];
    const bool shapes_ok = up.dims[0] == hidden && up.dims[1] == inter && up.dims[2] == experts &&
                           down.dims[0] == inter && down.dims[1] == hidden && down.dims[2] == experts &&
                           router.dims[0] == hidden && router.dims[1] == experts && router.dims[2] == 1 &&
                           up.type == gate.type && down.type == gate.type;
    if (!shapes_ok) {
        set_error(MMHIP_ERR_INVALID, p + "ffn_*: expert tensors disagree in shape or type");
        return MMHIP_ERR_INVALID;
    }
    mmhip_moe_weights w;
    std::memset(&w, 0, sizeof(w));
    w.hidden_size = (uint32_t)hidden;
    w.moe_intermediate = (uint32_t)inter;
    w.n_routed_experts = (uint32_t)experts;
    w.expert_type = gate.type;
    w.router_type = router.type;
    w.router_host = router.data;
    w.expert_gate_host = gate.data;
    w.expert_up_host = up.data;
    w.expert_down_host = down.data;
    w.shared_type = gate.type;
    w.shared_intermediate = (uint32_t)inter;
    // HyperParams.fromGguf (model.zig:107): routed_scaling_factor =
    // deepseek2.expert_weights_scale, default 1, whatever general.architecture says.
    w.routed_scaling_factor = 1.0f;
    {
        double s;
        if (mmhip_gguf_meta_float(g, "deepseek2.expert_weights_scale", &s) == MMHIP_OK) w.routed_scaling_factor = (float)s;
    }
    mmhip_gguf_tensor sg;
    if (mmhip_gguf_find_tensor(g, (p + "ffn_gate_shexp.weight").c_str(), &sg) == MMHIP_OK) {
        mmhip_gguf_tensor su, sd;
        if (int rc = tensor_matrix(g, p + "ffn_gate_shexp.weight", &sg)) return rc;
        if (int rc = tensor_matrix(g, p + "ffn_up_shexp.weight", &su)) return rc;
        if (int rc = tensor_matrix(g, p + "ffn_down_shexp.weight", &sd)) return rc;
        const uint64_t si = sg.dims[1];
        if (sg.dims[0] != hidden || sg.dims[2] != 1 || su.dims[0] != hidden || su.dims[1] != si ||
            su.dims[2] != 1 || sd.dims[0] != si || sd.dims[1] != hidden || sd.dims[2] != 1 ||
            su.type != sg.type || sd.type != sg.type) {
            set_error(MMHIP_ERR_INVALID, p + "ffn_*_shexp: shared expert tensors disagree in shape or type");
            return MMHIP_ERR_INVALID;
        }
        w.shared_type = sg.type;
        w.shared_intermediate = (uint32_t)si;
        w.shared_gate_host = sg.data;
        w.shared_up_host = su.data;
        w.shared_down_host = sd.data;
    }
    return mmhip_moe_layer_create(ctx, &w, out_layer);
}

}  // extern "C"
