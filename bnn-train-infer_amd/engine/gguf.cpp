// GGUF v3 reader: memory-maps the file, parses the metadata the engine needs and the
// tensor table, and checks every tensor's extent against the mapping.
//
// Accepts and rejects what the reference reader does (bnn-sw-v2/gguf.c:404-490):
// version 3 only, at most 4096 metadata entries, alignment 1..4096 (default 32),
// tensor types F32 (0), F16 (1) and Q1_0 (41, 18-byte blocks over [in, out] with
// in % 128 == 0), rank 1..4, non-empty tensor table, general.architecture present.
// Typed keys with the wrong type are format errors; unknown keys are skipped.
#include "engine_internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace bnne {
namespace {

enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};

// Little-endian reader over [p, end); any overrun clears ok and yields zeros.
struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    bool ok;

    bool need(uint64_t n) {
        if (!ok || n > (uint64_t)(end - p))
            ok = false;
        return ok;
    }
    uint64_t uint(unsigned bytes) {
        if (!need(bytes))
            return 0;
        uint64_t v = 0;
        for (unsigned i = 0; i < bytes; ++i)
            v |= (uint64_t)p[i] << (8 * i);
        p += bytes;
        return v;
    }
    uint32_t u32() { return (uint32_t)uint(4); }
    uint64_t u64() { return uint(8); }
    GgufString str() {
        GgufString s = {nullptr, 0};
        const uint64_t n = u64();
        if (!ok || n > UINT32_MAX || !need(n)) {
            ok = false;
            return s;
        }
        s.data = p;
        s.length = (uint32_t)n;
        p += n;
        return s;
    }
};

unsigned scalar_bytes(uint32_t type) {
    switch (type) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

bool skip(Reader& r, uint32_t type, unsigned depth) {
    if (!r.ok || depth > 4)
        return false;
    if (const unsigned n = scalar_bytes(type)) {
        r.uint(n);
        return r.ok;
    }
    if (type == kString) {
        r.str();
        return r.ok;
    }
    if (type != kArray)
        return false;
    const uint32_t element = r.u32();
    const uint64_t count = r.u64();
    for (uint64_t i = 0; r.ok && i < count; ++i)
        if (!skip(r, element, depth + 1))
            return false;
    return r.ok;
}

// Integer-typed value (any width, signed values sign-extended), as gguf.c:126-140.
bool read_integer(Reader& r, uint32_t type, uint64_t* out) {
    switch (type) {
    case kU8: case kBool: *out = r.uint(1); break;
    case kI8: *out = (uint64_t)(int64_t)(int8_t)r.uint(1); break;
    case kU16: *out = r.uint(2); break;
    case kI16: *out = (uint64_t)(int64_t)(int16_t)r.uint(2); break;
    case kU32: *out = r.uint(4); break;
    case kI32: *out = (uint64_t)(int64_t)(int32_t)r.uint(4); break;
    case kU64: case kI64: *out = r.uint(8); break;
    default: return false;
    }
    return r.ok;
}

bool read_float(Reader& r, uint32_t type, float* out) {
    if (type == kF32) {
        const uint32_t bits = r.u32();
        std::memcpy(out, &bits, 4);
    } else if (type == kF64) {
        const uint64_t bits = r.u64();
        double d;
        std::memcpy(&d, &bits, 8);
        *out = (float)d;
    } else {
        return false;
    }
    return r.ok && std::isfinite(*out);
}

bool read_text(Reader& r, uint32_t type, char* dst, size_t size) {
    if (type != kString)
        return false;
    const GgufString s = r.str();
    if (!r.ok)
        return false;
    const size_t n = s.length < size - 1 ? s.length : size - 1;
    std::memcpy(dst, s.data, n);
    dst[n] = '\0';
    return true;
}

bool key_is(const GgufString& key, const char* name) {
    const size_t n = std::strlen(name);
    return key.length == n && std::memcmp(key.data, name, n) == 0;
}

// "bnn-mlp.block.<decimal>.activation" -> index (gguf.c:168-186)
bool mlp_activation_index(const GgufString& key, uint32_t* index) {
    static const char pre[] = "bnn-mlp.block.", post[] = ".activation";
    const size_t np = sizeof pre - 1, ns = sizeof post - 1;
    if (key.length <= np + ns || std::memcmp(key.data, pre, np) != 0 ||
        std::memcmp(key.data + key.length - ns, post, ns) != 0)
        return false;
    uint64_t v = 0;
    for (size_t i = np; i < key.length - ns; ++i) {
        const uint8_t ch = key.data[i];
        if (ch < '0' || ch > '9' || v > 63)
            return false;
        v = v * 10 + (ch - '0');
    }
    *index = (uint32_t)v;
    return true;
}

BNNE_Status store_activation(Gguf* g, uint32_t index, Reader& r, uint32_t type) {
    if (type != kString)
        return BNNE_EFORMAT;
    if (index >= g->mlp_activation_count) {
        const uint64_t count = (uint64_t)index + 1;
        if (count > 64)
            return BNNE_EFORMAT;
        auto* grown = static_cast<char(*)[16]>(std::realloc(g->mlp_activations, count * sizeof *g->mlp_activations));
        if (!grown)
            return BNNE_ENOMEM;
        std::memset(grown + g->mlp_activation_count, 0, (count - g->mlp_activation_count) * sizeof *grown);
        g->mlp_activations = grown;
        g->mlp_activation_count = count;
    }
    return read_text(r, type, g->mlp_activations[index], sizeof g->mlp_activations[index]) ? BNNE_OK
                                                                                             : BNNE_EFORMAT;
}

// A string array: checked for type, counted, and (when 'keep' is given) its strings
// recorded as views into the mapping.  'seen' rejects a repeated key.
BNNE_Status string_array(Reader& r, uint32_t type, bool* seen, uint64_t* count_out, GgufString** keep = nullptr) {
    if (*seen || type != kArray)
        return BNNE_EFORMAT;
    *seen = true;
    const uint32_t element = r.u32();
    const uint64_t count = r.u64();
    if (!r.ok || element != kString || count > SIZE_MAX / sizeof(GgufString))
        return BNNE_EFORMAT;
    GgufString* out = nullptr;
    if (keep && count) {
        out = static_cast<GgufString*>(std::calloc(count, sizeof(GgufString)));
        if (!out)
            return BNNE_ENOMEM;
    }
    for (uint64_t i = 0; i < count; ++i) {
        const GgufString v = r.str();
        if (!r.ok) {
            std::free(out);
            return BNNE_EFORMAT;
        }
        if (out)
            out[i] = v;
    }
    if (keep)
        *keep = out;
    if (count_out)
        *count_out = count;
    return BNNE_OK;
}

BNNE_Status int_array(Reader& r, uint32_t type, bool* seen, uint32_t** out, uint64_t* count_out) {
    if (*seen || type != kArray)
        return BNNE_EFORMAT;
    *seen = true;
    const uint32_t element = r.u32();
    const uint64_t count = r.u64();
    if (!r.ok || (element != kI32 && element != kU32) || count > SIZE_MAX / 4)
        return BNNE_EFORMAT;
    if (!r.need(count * 4))
        return BNNE_EFORMAT;
    uint32_t* v = count ? static_cast<uint32_t*>(std::malloc(count * 4)) : nullptr;
    if (count && !v)
        return BNNE_ENOMEM;
    for (uint64_t i = 0; i < count; ++i)
        v[i] = r.u32();
    *out = v;
    *count_out = count;
    return BNNE_OK;
}

struct IntKey {
    const char* name;
    uint64_t Gguf::*field;
};
const IntKey kIntKeys[] = {
    {"qwen3.block_count", &Gguf::block_count},
    {"qwen3.context_length", &Gguf::context_length},
    {"qwen3.embedding_length", &Gguf::embedding_length},
    {"qwen3.feed_forward_length", &Gguf::feed_forward_length},
    {"qwen3.attention.head_count", &Gguf::head_count},
    {"qwen3.attention.head_count_kv", &Gguf::head_count_kv},
    {"qwen3.attention.key_length", &Gguf::key_length},
    {"qwen3.attention.value_length", &Gguf::value_length},
    {"qwen3.rope.scaling.original_context_length", &Gguf::rope_original_context},
    {"bnn-mlp.block_count", &Gguf::mlp_block_count},
    {"bnn-mlp.class_count", &Gguf::mlp_class_count},
    {"bnn-mlp.input_features", &Gguf::mlp_input_features},
    {"bnn-mlp.input_pixels", &Gguf::mlp_input_pixels},
};
struct FloatKey {
    const char* name;
    float Gguf::*field;
};
const FloatKey kFloatKeys[] = {
    {"qwen3.attention.layer_norm_rms_epsilon", &Gguf::rms_epsilon},
    {"qwen3.rope.freq_base", &Gguf::rope_freq_base},
    {"qwen3.rope.scaling.factor", &Gguf::rope_factor},
    {"bnn-mlp.input_mean", &Gguf::mlp_input_mean},
    {"bnn-mlp.input_std", &Gguf::mlp_input_std},
};

BNNE_Status parse_metadata(Reader& r, Gguf* g, uint64_t count) {
    if (!r.ok || count > 4096)
        return BNNE_EFORMAT;
    bool labels = false, tokens = false, types = false, merges = false;
    for (uint64_t i = 0; i < count; ++i) {
        const GgufString key = r.str();
        const uint32_t type = r.u32();
        if (!r.ok)
            return BNNE_EFORMAT;
        uint64_t v = 0;
        uint32_t index = 0;
        BNNE_Status st = BNNE_OK;
        bool handled = false;
        for (const IntKey& k : kIntKeys)
            if (key_is(key, k.name)) {
                if (!read_integer(r, type, &(g->*k.field)))
                    return BNNE_EFORMAT;
                handled = true;
            }
        for (const FloatKey& k : kFloatKeys)
            if (key_is(key, k.name)) {
                if (!read_float(r, type, &(g->*k.field)))
                    return BNNE_EFORMAT;
                handled = true;
            }
        if (handled)
            continue;
        if (key_is(key, "general.architecture")) {
            if (!read_text(r, type, g->architecture, sizeof g->architecture))
                return BNNE_EFORMAT;
        } else if (key_is(key, "general.alignment")) {
            if (!read_integer(r, type, &v) || v == 0 || v > 4096)
                return BNNE_EFORMAT;
            g->alignment = (uint32_t)v;
        } else if (key_is(key, "qwen3.rope.scaling.type")) {
            if (!read_text(r, type, g->rope_scaling_type, sizeof g->rope_scaling_type))
                return BNNE_EFORMAT;
        } else if (key_is(key, "bnn-mlp.labels")) {
            st = string_array(r, type, &labels, nullptr);
        } else if (mlp_activation_index(key, &index)) {
            st = store_activation(g, index, r, type);
        } else if (key_is(key, "tokenizer.ggml.model") || key_is(key, "tokenizer.ggml.pre")) {
            char scratch[32];
            if (!read_text(r, type, scratch, sizeof scratch))
                return BNNE_EFORMAT;
        } else if (key_is(key, "tokenizer.ggml.tokens")) {
            st = string_array(r, type, &tokens, &g->token_count, &g->tokens);
        } else if (key_is(key, "tokenizer.ggml.token_type")) {
            st = int_array(r, type, &types, &g->token_types, &g->token_type_count);
        } else if (key_is(key, "tokenizer.ggml.merges")) {
            st = string_array(r, type, &merges, nullptr);
        } else if (key_is(key, "tokenizer.ggml.eos_token_id")) {
            if (!read_integer(r, type, &v))
                return BNNE_EFORMAT;
            g->eos_token_id = (uint32_t)v;
            g->has_eos = 1;
        } else if (key_is(key, "tokenizer.ggml.bos_token_id")) {
            if (!read_integer(r, type, &v))
                return BNNE_EFORMAT;
            g->bos_token_id = (uint32_t)v;
            g->has_bos = 1;
        } else if (key_is(key, "tokenizer.ggml.padding_token_id") || key_is(key, "tokenizer.ggml.add_bos_token")) {
            if (!read_integer(r, type, &v))
                return BNNE_EFORMAT;
        } else if (!skip(r, type, 0)) {
            return BNNE_EFORMAT;
        }
        if (st != BNNE_OK)
            return st;
    }
    return r.ok ? BNNE_OK : BNNE_EFORMAT;
}

BNNE_Status parse_tensors(Reader& r, Gguf* g, uint64_t count) {
    if (!r.ok || count == 0 || count > SIZE_MAX / sizeof(GgufTensor))
        return BNNE_EFORMAT;
    g->tensors = static_cast<GgufTensor*>(std::calloc(count, sizeof(GgufTensor)));
    if (!g->tensors)
        return BNNE_ENOMEM;
    g->tensor_count = count;
    for (uint64_t i = 0; i < count; ++i) {
        GgufTensor& t = g->tensors[i];
        t.name = r.str();
        t.rank = r.u32();
        if (!r.ok || t.rank == 0 || t.rank > kMaxDims)
            return BNNE_EFORMAT;
        for (uint32_t d = 0; d < t.rank; ++d)
            t.dims[d] = r.u64();
        t.type = r.u32();
        t.offset = r.u64();
        if (!r.ok)
            return BNNE_EFORMAT;
    }
    return BNNE_OK;
}

BNNE_Status tensor_bytes(GgufTensor& t) {
    uint64_t count = 1;
    for (uint32_t d = 0; d < t.rank; ++d) {
        if (t.dims[d] == 0 || count > UINT64_MAX / t.dims[d])
            return BNNE_EFORMAT;
        count *= t.dims[d];
    }
    if (t.type == kTypeF32) {
        if (count > UINT64_MAX / 4)
            return BNNE_EFORMAT;
        t.bytes = count * 4;
    } else if (t.type == kTypeF16) {
        if (count > UINT64_MAX / 2)
            return BNNE_EFORMAT;
        t.bytes = count * 2;
    } else if (t.type == kTypeQ1_0) {
        if (t.rank != 2 || t.dims[0] % kGroup != 0 || t.dims[1] > UINT64_MAX / 18)
            return BNNE_EFORMAT;
        const uint64_t groups = t.dims[0] / kGroup;
        if (t.dims[1] > UINT64_MAX / groups)
            return BNNE_EFORMAT;
        t.bytes = t.dims[1] * groups * 18;
    } else {
        return BNNE_ENOTSUP;
    }
    return BNNE_OK;
}

}  // namespace

BNNE_Status gguf_open(const char* path, Gguf** out) {
    if (!path || !out)
        return BNNE_EINVAL;
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0)
        return error(BNNE_EIO, "%s: cannot open GGUF file", path);
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return error(BNNE_EIO, "%s: cannot stat GGUF file", path);
    }
    const size_t size = (size_t)st.st_size;
    void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED)
        return error(BNNE_EIO, "%s: cannot mmap GGUF file", path);

    Gguf* g = static_cast<Gguf*>(std::calloc(1, sizeof(Gguf)));
    if (!g) {
        ::munmap(map, size);
        return error(BNNE_ENOMEM, "out of memory");
    }
    g->mapping = static_cast<uint8_t*>(map);
    g->mapping_bytes = size;
    g->alignment = 32;

    Reader r = {g->mapping, g->mapping + size, true};
    const bool magic = r.need(4) && std::memcmp(r.p, "GGUF", 4) == 0;
    r.p += r.ok ? 4 : 0;
    const uint32_t version = r.u32();
    const uint64_t tensor_count = r.u64();
    const uint64_t metadata_count = r.u64();
    if (!r.ok || !magic || version != 3) {
        gguf_close(g);
        return error(BNNE_EFORMAT, "%s: unsupported GGUF header or version", path);
    }
    BNNE_Status status = parse_metadata(r, g, metadata_count);
    if (status == BNNE_OK)
        status = parse_tensors(r, g, tensor_count);
    if (status != BNNE_OK) {
        gguf_close(g);
        return error(status, "%s: invalid GGUF metadata or tensor table", path);
    }
    if (!g->architecture[0]) {
        gguf_close(g);
        return error(BNNE_EFORMAT, "%s: missing general.architecture", path);
    }
    const size_t info_end = (size_t)(r.p - g->mapping);
    const size_t align = g->alignment;
    g->data_offset = (info_end + align - 1) / align * align;
    if (g->data_offset > size) {
        gguf_close(g);
        return error(BNNE_EFORMAT, "%s: GGUF data section is out of bounds", path);
    }
    for (uint64_t i = 0; i < g->tensor_count; ++i) {
        GgufTensor& t = g->tensors[i];
        status = tensor_bytes(t);
        if (status != BNNE_OK) {
            gguf_close(g);
            return error(status, "%s: unsupported tensor type or shape", path);
        }
        const uint64_t available = size - g->data_offset;
        if (t.offset > available || t.bytes > available - t.offset) {
            gguf_close(g);
            return error(BNNE_EFORMAT, "%s: GGUF tensor data is out of bounds", path);
        }
    }
    if (g->rope_factor <= 0.0f)
        g->rope_factor = 1.0f;
    if (g->rope_original_context == 0)
        g->rope_original_context = g->context_length;
    *out = g;
    return BNNE_OK;
}

void gguf_close(Gguf* g) {
    if (!g)
        return;
    std::free(g->tensors);
    std::free(g->mlp_activations);
    std::free(g->tokens);
    std::free(g->token_types);
    if (g->mapping)
        ::munmap(g->mapping, g->mapping_bytes);
    std::free(g);
}

const GgufTensor* gguf_find(const Gguf* g, const char* name) {
    if (!g || !name)
        return nullptr;
    const size_t n = std::strlen(name);
    for (uint64_t i = 0; i < g->tensor_count; ++i) {
        const GgufTensor& t = g->tensors[i];
        if (t.name.length == n && std::memcmp(t.name.data, name, n) == 0)
            return &t;
    }
    return nullptr;
}

const uint8_t* gguf_data(const Gguf* g, const GgufTensor* t) {
    return g && t ? g->mapping + g->data_offset + t->offset : nullptr;
}

}  // namespace bnne
