// Token pieces and end-of-generation ids from the GGUF vocabulary
// (bnn-sw-v2/tokenizer/tokenizer-bpe.c:597-643 builds the same table).
//
// Byte-level BPE vocabularies spell every byte b as one code point: b itself for the
// printable bytes 33..126, 161..172 and 174..255, and 256 + n for the n-th of the
// remaining bytes.  A token's piece is its text with each such code point replaced
// by its byte (other text is kept as is); control and user-defined tokens (types 3
// and 4) keep their text.  The vocabulary must spell all 256 bytes.  End of
// generation: the declared EOS id and the tokens "<|endoftext|>" and "<|im_end|>".
// Text encoding (BNNE_Tokenize) is not part of this build.
#include "engine_internal.h"

#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_set>

namespace bnne {
namespace {

void byte_code_points(uint32_t cp_of[256]) {
    uint32_t extra = 0;
    for (uint32_t b = 0; b < 256; ++b) {
        const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || b >= 174;
        cp_of[b] = printable ? b : 256 + extra++;
    }
}

// One well-formed UTF-8 sequence at p (Unicode 3.9, table 3-7); 0 if none.
size_t utf8_next(const uint8_t* p, size_t n, uint32_t* cp) {
    if (!n)
        return 0;
    const uint8_t b0 = p[0];
    auto cont = [&](size_t i) { return i < n && (p[i] & 0xc0) == 0x80; };
    if (b0 < 0x80) {
        *cp = b0;
        return 1;
    }
    if (b0 >= 0xc2 && b0 <= 0xdf && cont(1)) {
        *cp = ((uint32_t)(b0 & 0x1f) << 6) | (p[1] & 0x3f);
        return 2;
    }
    if (b0 >= 0xe0 && b0 <= 0xef && cont(1) && cont(2)) {
        const uint32_t v = ((uint32_t)(b0 & 0x0f) << 12) | ((uint32_t)(p[1] & 0x3f) << 6) | (p[2] & 0x3f);
        if (v < 0x800 || (v >= 0xd800 && v <= 0xdfff))
            return 0;
        *cp = v;
        return 3;
    }
    if (b0 >= 0xf0 && b0 <= 0xf4 && cont(1) && cont(2) && cont(3)) {
        const uint32_t v = ((uint32_t)(b0 & 0x07) << 18) | ((uint32_t)(p[1] & 0x3f) << 12) |
                           ((uint32_t)(p[2] & 0x3f) << 6) | (p[3] & 0x3f);
        if (v < 0x10000 || v > 0x10ffff)
            return 0;
        *cp = v;
        return 4;
    }
    return 0;
}

std::string utf8_of(uint32_t cp) {
    std::string s;
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xc0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3f));
    } else {
        s += (char)(0xe0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3f));
        s += (char)(0x80 | (cp & 0x3f));
    }
    return s;
}

}  // namespace

void vocab_free(Vocab* v) {
    if (!v)
        return;
    std::free(v->text);
    std::free(v->off);
    std::free(v->len);
    std::free(v);
}

BNNE_Status vocab_build(const Gguf* g, Vocab** out) {
    *out = nullptr;
    if (!g->tokens || !g->token_count)
        return error(BNNE_EFORMAT, "tokenizer has no vocabulary");
    if (g->token_count > UINT32_MAX)
        return error(BNNE_ERANGE, "tokenizer vocabulary is too large");
    uint32_t cp_of[256];
    byte_code_points(cp_of);
    {
        std::unordered_set<std::string> spelled;
        spelled.reserve(g->token_count * 2);
        for (uint64_t i = 0; i < g->token_count; ++i)
            spelled.emplace(reinterpret_cast<const char*>(g->tokens[i].data), g->tokens[i].length);
        for (uint32_t b = 0; b < 256; ++b)
            if (!spelled.count(utf8_of(cp_of[b])))
                return error(BNNE_EFORMAT, "vocabulary is missing a byte token");
    }
    int byte_of_cp[512];
    std::memset(byte_of_cp, 0xff, sizeof byte_of_cp);
    for (uint32_t b = 0; b < 256; ++b)
        byte_of_cp[cp_of[b]] = (int)b;

    Vocab* v = static_cast<Vocab*>(std::calloc(1, sizeof(Vocab)));
    uint64_t total = 0;
    for (uint64_t i = 0; i < g->token_count; ++i)
        total += g->tokens[i].length + 1u;
    if (v) {
        v->text = static_cast<char*>(std::malloc(total));
        v->off = static_cast<uint32_t*>(std::malloc(g->token_count * sizeof(uint32_t)));
        v->len = static_cast<uint32_t*>(std::malloc(g->token_count * sizeof(uint32_t)));
    }
    if (!v || !v->text || !v->off || !v->len || total > UINT32_MAX) {
        vocab_free(v);
        return error(total > UINT32_MAX ? BNNE_ERANGE : BNNE_ENOMEM, "vocabulary table");
    }
    v->count = g->token_count;
    size_t used = 0;
    for (uint64_t i = 0; i < g->token_count; ++i) {
        const GgufString& t = g->tokens[i];
        const uint32_t type = g->token_types && i < g->token_type_count ? g->token_types[i] : 1u;
        v->off[i] = (uint32_t)used;
        if (type == 3 || type == 4) {
            std::memcpy(v->text + used, t.data, t.length);
            used += t.length;
        } else {
            size_t pos = 0;
            while (pos < t.length) {
                uint32_t cp = 0;
                size_t n = utf8_next(t.data + pos, t.length - pos, &cp);
                if (n && cp < 512 && byte_of_cp[cp] >= 0) {
                    v->text[used++] = (char)byte_of_cp[cp];
                } else {
                    n = n ? n : 1;
                    std::memcpy(v->text + used, t.data + pos, n);
                    used += n;
                }
                pos += n;
            }
        }
        v->len[i] = (uint32_t)(used - v->off[i]);
        v->text[used++] = '\0';
    }
    auto add_eog = [&](uint32_t id) {
        for (uint32_t k = 0; k < v->n_eog; ++k)
            if (v->eog[k] == id)
                return;
        if (v->n_eog < 8)
            v->eog[v->n_eog++] = id;
    };
    if (g->has_eos && g->eos_token_id < g->token_count)
        add_eog(g->eos_token_id);
    for (uint64_t i = 0; i < g->token_count; ++i) {
        const GgufString& t = g->tokens[i];
        if ((t.length == 13 && std::memcmp(t.data, "<|endoftext|>", 13) == 0) ||
            (t.length == 10 && std::memcmp(t.data, "<|im_end|>", 10) == 0))
            add_eog((uint32_t)i);
    }
    *out = v;
    return BNNE_OK;
}

}  // namespace bnne
