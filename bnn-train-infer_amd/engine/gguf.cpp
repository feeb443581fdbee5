// GGUF v3 files: memory-mapped, indexed once, values decoded on request.
//
// What is accepted follows the reference reader (bnn-sw-v2/gguf.c:404-490), whose
// files and statuses callers share: version 3 only; at most 4096 metadata entries;
// values nest at most four arrays deep; general.alignment in 1..4096 (default 32);
// tensor ranks 1..4 and types F32 (0), F16 (1) and Q1_0 (41, 18-byte blocks over
// [in, out] with in % 128 == 0); a non-empty tensor table; general.architecture
// present; every tensor inside the data section.  The keys this engine reads have a
// fixed kind (integer, real, text, text array, word array) and a present key of the
// wrong kind -- or a repeated array key -- makes the file malformed.
#include "engine.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>

namespace bnne {
namespace {

// GGUF value types
enum : uint32_t {
    tU8 = 0, tI8 = 1, tU16 = 2, tI16 = 3, tU32 = 4, tI32 = 5, tF32 = 6, tBool = 7,
    tString = 8, tArray = 9, tU64 = 10, tI64 = 11, tF64 = 12
};

constexpr uint64_t kMaxEntries = 4096;
constexpr unsigned kMaxNesting = 4;

unsigned fixed_size(uint32_t type) {
    switch (type) {
    case tU8: case tI8: case tBool: return 1;
    case tU16: case tI16: return 2;
    case tU32: case tI32: case tF32: return 4;
    case tU64: case tI64: case tF64: return 8;
    default: return 0;
    }
}

uint64_t le(const uint8_t* p, unsigned n) {
    uint64_t v = 0;
    for (unsigned i = 0; i < n; ++i)
        v |= (uint64_t)p[i] << (8 * i);
    return v;
}

// A forward-only view of [at, end).  Every read checks its own bounds; a failed read
// leaves `at` at null, after which all reads fail.
struct Bytes {
    const uint8_t* at;
    const uint8_t* end;

    bool have(uint64_t n) const { return at && n <= (uint64_t)(end - at); }
    uint64_t take(unsigned n) {
        if (!have(n)) {
            at = nullptr;
            return 0;
        }
        const uint64_t v = le(at, n);
        at += n;
        return v;
    }
    std::string_view string() {
        const uint64_t n = take(8);
        if (n > UINT32_MAX || !have(n)) {
            at = nullptr;
            return {};
        }
        const std::string_view s(reinterpret_cast<const char*>(at), (size_t)n);
        at += n;
        return s;
    }
    // moves past one value of `type`; false for an unknown type or too deep a nesting
    bool skip(uint32_t type, unsigned depth) {
        if (!at || depth > kMaxNesting)
            return false;
        if (const unsigned n = fixed_size(type)) {
            take(n);
        } else if (type == tString) {
            string();
        } else if (type == tArray) {
            const uint32_t element = (uint32_t)take(4);
            const uint64_t count = take(8);
            if (const unsigned n = fixed_size(element)) {  // a block of fixed-size elements
                if (!at || count > UINT64_MAX / n || !have(count * n))
                    return at = nullptr, false;
                at += count * n;
                return true;
            }
            for (uint64_t i = 0; at && i < count; ++i)
                if (!skip(element, depth + 1))
                    return false;
        } else {
            return false;
        }
        return at != nullptr;
    }
};

[[noreturn]] void malformed(const char* path, const char* what) { raise(BNNE_EFORMAT, "%s: %s", path, what); }

// The kinds of the keys this engine reads.
enum class Kind { Integer, Real, Text, Texts, Words };

struct KnownKey {
    const char* key;
    Kind kind;
};
const KnownKey kKnownKeys[] = {
    {"general.architecture", Kind::Text},
    {"general.alignment", Kind::Integer},
    {"qwen3.block_count", Kind::Integer},
    {"qwen3.context_length", Kind::Integer},
    {"qwen3.embedding_length", Kind::Integer},
    {"qwen3.feed_forward_length", Kind::Integer},
    {"qwen3.attention.head_count", Kind::Integer},
    {"qwen3.attention.head_count_kv", Kind::Integer},
    {"qwen3.attention.key_length", Kind::Integer},
    {"qwen3.attention.value_length", Kind::Integer},
    {"qwen3.attention.layer_norm_rms_epsilon", Kind::Real},
    {"qwen3.rope.freq_base", Kind::Real},
    {"qwen3.rope.scaling.type", Kind::Text},
    {"qwen3.rope.scaling.factor", Kind::Real},
    {"qwen3.rope.scaling.original_context_length", Kind::Integer},
    {"bnn-mlp.block_count", Kind::Integer},
    {"bnn-mlp.class_count", Kind::Integer},
    {"bnn-mlp.input_features", Kind::Integer},
    {"bnn-mlp.input_pixels", Kind::Integer},
    {"bnn-mlp.input_mean", Kind::Real},
    {"bnn-mlp.input_std", Kind::Real},
    {"bnn-mlp.labels", Kind::Texts},
    {"tokenizer.ggml.model", Kind::Text},
    {"tokenizer.ggml.pre", Kind::Text},
    {"tokenizer.ggml.tokens", Kind::Texts},
    {"tokenizer.ggml.token_type", Kind::Words},
    {"tokenizer.ggml.merges", Kind::Texts},
    {"tokenizer.ggml.eos_token_id", Kind::Integer},
    {"tokenizer.ggml.bos_token_id", Kind::Integer},
    {"tokenizer.ggml.padding_token_id", Kind::Integer},
    {"tokenizer.ggml.add_bos_token", Kind::Integer},
};

// "bnn-mlp.block.<i>.activation" with i in decimal: its block index (capped at 1000).
std::optional<uint32_t> activation_index(std::string_view key) {
    constexpr std::string_view head = "bnn-mlp.block.", tail = ".activation";
    if (key.size() <= head.size() + tail.size() || key.substr(0, head.size()) != head ||
        key.substr(key.size() - tail.size()) != tail)
        return std::nullopt;
    uint32_t index = 0;
    for (char ch : key.substr(head.size(), key.size() - head.size() - tail.size())) {
        if (ch < '0' || ch > '9')
            return std::nullopt;
        index = index * 10u + (uint32_t)(ch - '0');
        if (index > 1000u)
            index = 1000u;
    }
    return index;
}
bool is_activation_key(std::string_view key) { return activation_index(key).has_value(); }

std::optional<Kind> kind_of(std::string_view key) {
    for (const KnownKey& k : kKnownKeys)
        if (key == k.key)
            return k.kind;
    if (is_activation_key(key))
        return Kind::Text;
    return std::nullopt;
}

// Integer value of a scalar entry (any integer type); false for other types.
bool decode_integer(const GgufFile::Entry& e, uint64_t* out) {
    const uint8_t* p = e.value;
    switch (e.type) {
    case tU8: case tBool: *out = p[0]; return true;
    case tI8: *out = (uint64_t)(int64_t)(int8_t)p[0]; return true;
    case tU16: *out = le(p, 2); return true;
    case tI16: *out = (uint64_t)(int64_t)(int16_t)le(p, 2); return true;
    case tU32: *out = le(p, 4); return true;
    case tI32: *out = (uint64_t)(int64_t)(int32_t)le(p, 4); return true;
    case tU64: case tI64: *out = le(p, 8); return true;
    default: return false;
    }
}

bool decode_real(const GgufFile::Entry& e, float* out) {
    if (e.type == tF32) {
        const uint32_t bits = (uint32_t)le(e.value, 4);
        std::memcpy(out, &bits, 4);
    } else if (e.type == tF64) {
        const uint64_t bits = le(e.value, 8);
        double d;
        std::memcpy(&d, &bits, 8);
        *out = (float)d;
    } else {
        return false;
    }
    return std::isfinite(*out);
}

// Element type and count of an array entry.
bool array_header(const GgufFile::Entry& e, uint32_t* element, uint64_t* count) {
    if (e.type != tArray)
        return false;
    *element = (uint32_t)le(e.value, 4);
    *count = le(e.value + 4, 8);
    return true;
}

bool entry_has_kind(const GgufFile::Entry& e, Kind kind) {
    uint64_t v;
    float f;
    uint32_t element;
    uint64_t count;
    switch (kind) {
    case Kind::Integer: return decode_integer(e, &v);
    case Kind::Real: return decode_real(e, &f);
    case Kind::Text: return e.type == tString;
    case Kind::Texts: return array_header(e, &element, &count) && element == tString;
    case Kind::Words: return array_header(e, &element, &count) && (element == tI32 || element == tU32);
    }
    return false;
}

// Bytes of a tensor's data; throws for types this engine does not read or bad shapes.
uint64_t tensor_bytes(const TensorRef& t, const char* path) {
    uint64_t elements = 1;
    for (uint32_t d = 0; d < t.rank; ++d) {
        if (t.dims[d] == 0 || elements > UINT64_MAX / t.dims[d])
            malformed(path, "tensor with an empty or overflowing shape");
        elements *= t.dims[d];
    }
    switch (t.type) {
    case kF32:
        if (elements > UINT64_MAX / 4)
            malformed(path, "tensor too large");
        return elements * 4;
    case kF16:
        if (elements > UINT64_MAX / 2)
            malformed(path, "tensor too large");
        return elements * 2;
    case kQ1_0: {
        if (t.rank != 2 || t.dims[0] % kGroup != 0)
            malformed(path, "Q1_0 tensor that is not [in, out] with in a multiple of 128");
        const uint64_t blocks_per_row = t.dims[0] / kGroup;
        if (t.dims[1] > UINT64_MAX / 18 / blocks_per_row)
            malformed(path, "tensor too large");
        return t.dims[1] * blocks_per_row * 18;
    }
    default:
        raise(BNNE_ENOTSUP, "%s: tensor '%.*s' has type %u (F32, F16 and Q1_0 are read)", path, (int)t.name.size(),
              t.name.data(), t.type);
    }
}

}  // namespace

std::unique_ptr<GgufFile> GgufFile::open(const char* path) {
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0)
        raise(BNNE_EIO, "%s: cannot be opened", path);
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        raise(BNNE_EIO, "%s: empty or unreadable", path);
    }
    void* map = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED)
        raise(BNNE_EIO, "%s: cannot be mapped", path);
    std::unique_ptr<GgufFile> f(new GgufFile);
    f->map_ = map;
    f->map_bytes_ = (size_t)st.st_size;

    const uint8_t* base = static_cast<const uint8_t*>(map);
    Bytes in{base, base + f->map_bytes_};
    const bool magic = in.have(4) && std::memcmp(in.at, "GGUF", 4) == 0;
    in.take(4);
    const uint32_t version = (uint32_t)in.take(4);
    const uint64_t n_tensors = in.take(8), n_entries = in.take(8);
    if (!in.at || !magic || version != 3)
        malformed(path, "not a GGUF version 3 file");
    if (n_entries > kMaxEntries)
        malformed(path, "too many metadata entries");

    f->entries_.reserve((size_t)n_entries);
    for (uint64_t i = 0; i < n_entries; ++i) {
        Entry e;
        e.key = in.string();
        e.type = (uint32_t)in.take(4);
        e.value = in.at;
        if (!in.skip(e.type, 0))
            malformed(path, "truncated or malformed metadata");
        e.end = in.at;
        f->entries_.push_back(e);
    }
    // a tensor record takes at least 32 bytes (name length, rank, one dimension, type,
    // offset): a count the rest of the file cannot hold is malformed, not an allocation
    if (n_tensors == 0)
        malformed(path, "no tensor table");
    if (!in.at || n_tensors > (uint64_t)(in.end - in.at) / 32u)
        malformed(path, "tensor table longer than the file");
    f->tensors_.reserve((size_t)n_tensors);
    std::vector<uint64_t> offsets;  // relative to the data section, whose start is known later
    offsets.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorRef t{};
        t.name = in.string();
        t.rank = (uint32_t)in.take(4);
        if (!in.at || t.rank == 0 || t.rank > 4)
            malformed(path, "truncated tensor table or tensor rank outside 1..4");
        for (uint32_t d = 0; d < t.rank; ++d)
            t.dims[d] = in.take(8);
        t.type = (uint32_t)in.take(4);
        const uint64_t offset = in.take(8);
        if (!in.at)
            malformed(path, "truncated tensor table");
        offsets.push_back(offset);
        f->tensors_.push_back(t);
    }

    // the keys this engine reads: usable kind, arrays not repeated
    std::vector<std::string_view> arrays_seen;
    for (const Entry& e : f->entries_) {
        const std::optional<Kind> kind = kind_of(e.key);
        if (!kind)
            continue;
        if (!entry_has_kind(e, *kind))
            raise(BNNE_EFORMAT, "%s: metadata '%.*s' has the wrong type", path, (int)e.key.size(), e.key.data());
        if (*kind == Kind::Texts || *kind == Kind::Words) {
            for (std::string_view seen : arrays_seen)
                if (seen == e.key)
                    raise(BNNE_EFORMAT, "%s: metadata '%.*s' appears twice", path, (int)e.key.size(), e.key.data());
            arrays_seen.push_back(e.key);
        }
    }
    for (const Entry& e : f->entries_)
        if (activation_index(e.key).value_or(0) > 63u)
            malformed(path, "activation of a bnn-mlp block beyond the 64th");
    const std::optional<std::string_view> arch = f->text("general.architecture");
    if (!arch || arch->empty())
        malformed(path, "general.architecture is missing");
    f->architecture_.assign(arch->data(), arch->size());
    uint64_t alignment = f->integer("general.alignment").value_or(32);
    if (alignment == 0 || alignment > 4096)
        malformed(path, "general.alignment outside 1..4096");

    // the data section starts at the next multiple of the alignment
    const uint64_t header_end = (uint64_t)(in.at - base);
    const uint64_t data_start = (header_end + alignment - 1) / alignment * alignment;
    if (data_start > f->map_bytes_)
        malformed(path, "data section beyond the end of the file");
    const uint64_t room = f->map_bytes_ - data_start;
    for (size_t i = 0; i < f->tensors_.size(); ++i) {
        TensorRef& t = f->tensors_[i];
        const uint64_t offset = offsets[i];
        t.bytes = tensor_bytes(t, path);
        if (offset > room || t.bytes > room - offset)
            malformed(path, "tensor data beyond the end of the file");
        t.data = base + data_start + offset;
    }
    return f;
}

GgufFile::~GgufFile() {
    if (map_)
        ::munmap(map_, map_bytes_);
}

const GgufFile::Entry* GgufFile::entry(std::string_view key) const {
    for (auto it = entries_.rbegin(); it != entries_.rend(); ++it)
        if (it->key == key)
            return &*it;
    return nullptr;
}

bool GgufFile::has(std::string_view key) const { return entry(key) != nullptr; }

const TensorRef* GgufFile::tensor(std::string_view name) const {
    for (const TensorRef& t : tensors_)
        if (t.name == name)
            return &t;
    return nullptr;
}

std::optional<uint64_t> GgufFile::integer(std::string_view key) const {
    const Entry* e = entry(key);
    uint64_t v;
    if (!e)
        return std::nullopt;
    if (!decode_integer(*e, &v))
        raise(BNNE_EFORMAT, "metadata '%.*s' is not an integer", (int)key.size(), key.data());
    return v;
}

std::optional<float> GgufFile::real(std::string_view key) const {
    const Entry* e = entry(key);
    float v;
    if (!e)
        return std::nullopt;
    if (!decode_real(*e, &v))
        raise(BNNE_EFORMAT, "metadata '%.*s' is not a finite real", (int)key.size(), key.data());
    return v;
}

std::optional<std::string_view> GgufFile::text(std::string_view key) const {
    const Entry* e = entry(key);
    if (!e)
        return std::nullopt;
    if (e->type != tString)
        raise(BNNE_EFORMAT, "metadata '%.*s' is not a string", (int)key.size(), key.data());
    Bytes b{e->value, e->end};
    return b.string();
}

std::vector<std::string_view> GgufFile::texts(std::string_view key) const {
    std::vector<std::string_view> out;
    const Entry* e = entry(key);
    uint32_t element;
    uint64_t count;
    if (!e)
        return out;
    if (!array_header(*e, &element, &count) || element != tString)
        raise(BNNE_EFORMAT, "metadata '%.*s' is not a string array", (int)key.size(), key.data());
    Bytes b{e->value + 12, e->end};
    out.reserve((size_t)count);
    for (uint64_t i = 0; i < count; ++i)
        out.push_back(b.string());
    return out;
}

std::vector<uint32_t> GgufFile::words(std::string_view key) const {
    std::vector<uint32_t> out;
    const Entry* e = entry(key);
    uint32_t element;
    uint64_t count;
    if (!e)
        return out;
    if (!array_header(*e, &element, &count) || (element != tI32 && element != tU32))
        raise(BNNE_EFORMAT, "metadata '%.*s' is not a 32-bit integer array", (int)key.size(), key.data());
    out.resize((size_t)count);
    for (uint64_t i = 0; i < count; ++i)
        out[i] = (uint32_t)le(e->value + 12 + 4 * i, 4);
    return out;
}

std::vector<float> read_floats(const GgufFile& file, std::string_view name, size_t count) {
    const TensorRef* t = file.tensor(name);
    if (!t || (t->type != kF32 && t->type != kF16))
        raise(BNNE_EFORMAT, "no F32/F16 tensor '%.*s'", (int)name.size(), name.data());
    const uint64_t elements = t->bytes / (t->type == kF32 ? 4u : 2u);
    if (elements != count)
        raise(BNNE_EFORMAT, "tensor '%.*s' holds %llu values where %zu belong", (int)name.size(), name.data(),
              (unsigned long long)elements, count);
    std::vector<float> v(count);
    for (size_t i = 0; i < count; ++i) {
        if (t->type == kF32) {
            const uint32_t bits = (uint32_t)le(t->data + 4 * i, 4);
            std::memcpy(&v[i], &bits, 4);
        } else {
            v[i] = half_to_float((uint16_t)le(t->data + 2 * i, 2));
        }
        if (!std::isfinite(v[i]))
            raise(BNNE_EFORMAT, "tensor '%.*s' holds a NaN or infinity", (int)name.size(), name.data());
    }
    return v;
}

}  // namespace bnne
