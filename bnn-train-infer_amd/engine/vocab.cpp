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
#include "engine.hpp"

#include <cstring>
#include <optional>
#include <string>
#include <string_view>
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

Vocab::Vocab(const GgufFile& file) {
    const std::vector<std::string_view> tokens = file.texts("tokenizer.ggml.tokens");
    const std::vector<uint32_t> types = file.words("tokenizer.ggml.token_type");
    if (tokens.empty())
        raise(BNNE_EFORMAT, "the model has no token list");
    if (tokens.size() > UINT32_MAX)
        raise(BNNE_ERANGE, "the token list is too long");
    uint32_t cp_of[256];
    byte_code_points(cp_of);
    {
        std::unordered_set<std::string_view> spelled(tokens.begin(), tokens.end());
        for (uint32_t b = 0; b < 256; ++b)
            if (!spelled.count(utf8_of(cp_of[b])))
                raise(BNNE_EFORMAT, "the token list does not spell every byte");
    }
    int byte_of_cp[512];
    std::memset(byte_of_cp, 0xff, sizeof byte_of_cp);
    for (uint32_t b = 0; b < 256; ++b)
        byte_of_cp[cp_of[b]] = (int)b;

    offset_.resize(tokens.size());
    length_.resize(tokens.size());
    for (size_t i = 0; i < tokens.size(); ++i) {
        const std::string_view t = tokens[i];
        const uint8_t* p = reinterpret_cast<const uint8_t*>(t.data());
        const uint32_t type = i < types.size() ? types[i] : 1u;
        if (text_.size() > UINT32_MAX - t.size() - 1)
            raise(BNNE_ERANGE, "the token list is too long");
        offset_[i] = (uint32_t)text_.size();
        if (type == 3 || type == 4) {  // control and user-defined tokens keep their text
            text_.append(t);
        } else {
            size_t pos = 0;
            while (pos < t.size()) {
                uint32_t cp = 0;
                size_t n = utf8_next(p + pos, t.size() - pos, &cp);
                if (n && cp < 512 && byte_of_cp[cp] >= 0) {
                    text_.push_back((char)byte_of_cp[cp]);
                } else {
                    n = n ? n : 1;
                    text_.append(t.substr(pos, n));
                }
                pos += n;
            }
        }
        length_[i] = (uint32_t)(text_.size() - offset_[i]);
        text_.push_back('\0');
    }
    const auto add_eog = [&](uint32_t id) {
        for (uint32_t e : eog_)
            if (e == id)
                return;
        if (eog_.size() < 8)
            eog_.push_back(id);
    };
    if (const std::optional<uint64_t> eos = file.integer("tokenizer.ggml.eos_token_id"))
        if ((uint32_t)*eos < tokens.size())
            add_eog((uint32_t)*eos);
    for (size_t i = 0; i < tokens.size(); ++i)
        if (tokens[i] == "<|endoftext|>" || tokens[i] == "<|im_end|>")
            add_eog((uint32_t)i);
}

std::string_view Vocab::piece(uint32_t id) const { return std::string_view(text_.data() + offset_[id], length_[id]); }

bool Vocab::ends_generation(uint32_t id) const {
    for (uint32_t e : eog_)
        if (e == id)
            return true;
    return false;
}

}  // namespace bnne
