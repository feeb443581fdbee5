// The shared linear operator: Q1_0 tensors -> BNN_Matrix chunks -> BNN_Execute.
//
// Q1_0 storage (linear.c:26-62): a tensor of dims [in, out] is out x (in/128) blocks of
// 18 bytes, each an fp16 scale (little-endian) followed by 16 bytes of sign bits, LSB
// first.  The accelerator layout wants bits[out][in/8] and scales[out][in/128], so the
// blocks are split; a non-finite scale is a format error.
//
// Chunking (linear.c:90-131): outputs are split into ceil(out / max_out_features)
// matrices; the forward pass is one BufferWrite of the F32 input, then per chunk one
// GEMV_F32 BNN_Execute and one BufferRead into y[out_off..] (linear.c:161-216), with
// the same statistics bookkeeping.
#include "engine_internal.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace bnne {

namespace {
void* alloc_array(size_t count, size_t size) {
    if (!count || size > SIZE_MAX / count)
        return nullptr;
    return std::malloc(count * size);
}
uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
}  // namespace

BNNE_Status q1_0_read(const Gguf* g, const char* tensor, uint32_t in, uint32_t out, uint8_t** out_bits,
                      uint16_t** out_scales) {
    const GgufTensor* t = gguf_find(g, tensor);
    if (!t || t->type != kTypeQ1_0 || t->rank != 2 || t->dims[0] != in || t->dims[1] != out || in % kGroup != 0 ||
        t->bytes != (uint64_t)out * (in / kGroup) * 18)
        return error(BNNE_EFORMAT, "unexpected Q1_0 tensor '%s' shape or type", tensor);
    const size_t row_bytes = in / 8u, groups = in / kGroup;
    auto* bits = static_cast<uint8_t*>(alloc_array(out, row_bytes));
    auto* scales = static_cast<uint16_t*>(alloc_array((size_t)out * groups, sizeof(uint16_t)));
    if (!bits || !scales) {
        std::free(bits);
        std::free(scales);
        return error(BNNE_ENOMEM, "out of memory");
    }
    const uint8_t* src = gguf_data(g, t);
    for (size_t o = 0; o < out; ++o) {
        for (size_t grp = 0; grp < groups; ++grp) {
            const uint8_t* block = src + (o * groups + grp) * 18;
            const uint16_t scale = le16(block);
            if (!std::isfinite(fp16_to_fp32(scale))) {
                std::free(bits);
                std::free(scales);
                return error(BNNE_EFORMAT, "Q1_0 scale in '%s' is not finite", tensor);
            }
            scales[o * groups + grp] = scale;
            std::memcpy(bits + o * row_bytes + grp * 16, block + 2, 16);
        }
    }
    *out_bits = bits;
    *out_scales = scales;
    return BNNE_OK;
}

BNNE_Status linear_init(bnne_model* m, uint32_t in, uint32_t out, const uint8_t* bits, const uint16_t* scales,
                        Linear* l) {
    if (!m || !l || !bits || !scales || in == 0 || out == 0)
        return BNNE_EINVAL;
    std::memset(l, 0, sizeof *l);
    l->in = in;
    l->out = out;
    if (m->caps.group_size != kGroup || !(m->caps.supported_ops & BNN_CAP_GEMV_F32))
        return error(BNNE_ENOTSUP, "Q1_0 requires group size 128 and F32 GEMV support");
    if (in % kGroup != 0)
        return error(BNNE_EFORMAT, "Q1_0 input width is not group aligned");
    const uint32_t max_in = m->caps.max_in_features, max_out = m->caps.max_out_features;
    if (!max_in || !max_out)
        return error(BNNE_ENOTSUP, "accelerator does not report matrix limits");
    if (in > max_in)
        return error(BNNE_ENOTSUP, "Q1_0 input width %u exceeds accelerator limit %u", in, max_in);

    const uint32_t count = out / max_out + (out % max_out != 0);
    l->chunks = static_cast<LinearChunk*>(std::calloc(count, sizeof(LinearChunk)));
    if (!l->chunks)
        return error(BNNE_ENOMEM, "out of memory");
    l->n_chunks = count;
    const size_t row_bytes = in / 8u, groups = in / kGroup;
    for (uint32_t c = 0; c < count; ++c) {
        LinearChunk& ch = l->chunks[c];
        ch.out_off = c * max_out;
        ch.out_len = out - ch.out_off < max_out ? out - ch.out_off : max_out;
        BNN_MatrixDesc desc = {};
        desc.in_features = in;
        desc.out_features = ch.out_len;
        desc.group_size = kGroup;
        desc.weight_bits = bits + (size_t)ch.out_off * row_bytes;
        desc.weight_bytes = (size_t)ch.out_len * row_bytes;
        desc.scale_fp16 = scales + (size_t)ch.out_off * groups;
        desc.scale_count = (size_t)ch.out_len * groups;
        const BNN_Status st = BNN_MatrixCreate(m->device, &desc, &ch.matrix);
        if (st != BNN_OK) {
            linear_free(l);
            return accel_error(st, "BNN_MatrixCreate(Q1_0)");
        }
    }
    m->max_in = m->max_in > in ? m->max_in : in;
    const uint32_t chunk_max = out < max_out ? out : max_out;
    m->max_out = m->max_out > chunk_max ? m->max_out : chunk_max;
    return BNNE_OK;
}

BNNE_Status linear_load(bnne_model* m, const Gguf* g, const char* tensor, Linear* l) {
    const GgufTensor* t = gguf_find(g, tensor);
    if (!t || t->rank != 2 || t->dims[0] == 0 || t->dims[1] == 0 || t->dims[0] > UINT32_MAX ||
        t->dims[1] > UINT32_MAX)
        return error(BNNE_EFORMAT, "missing or invalid Q1_0 tensor '%s'", tensor);
    const uint32_t in = (uint32_t)t->dims[0], out = (uint32_t)t->dims[1];
    uint8_t* bits = nullptr;
    uint16_t* scales = nullptr;
    BNNE_Status st = q1_0_read(g, tensor, in, out, &bits, &scales);
    if (st == BNNE_OK)
        st = linear_init(m, in, out, bits, scales, l);
    std::free(bits);
    std::free(scales);
    return st;
}

void linear_free(Linear* l) {
    if (!l)
        return;
    for (uint32_t i = 0; i < l->n_chunks; ++i)
        BNN_MatrixDestroy(l->chunks[i].matrix);
    std::free(l->chunks);
    std::memset(l, 0, sizeof *l);
}

BNNE_Status linear_forward(bnne_context* c, const Linear* l, const float* x, float* y) {
    if (!c || !l || !x || !y || !c->in_buf || !c->out_buf)
        return BNNE_EINVAL;
    const bool stats = c->params.enable_stats != 0;
    const size_t in_bytes = (size_t)l->in * sizeof(float);
    uint64_t t0 = stats ? now_ns() : 0;
    BNNE_Status st = accel_error(BNN_BufferWrite(c->in_buf, 0, x, in_bytes), "BNN_BufferWrite");
    if (stats) {
        c->stats.transfer_ns += now_ns() - t0;
        c->stats.bytes_written += in_bytes;
    }
    if (st != BNNE_OK)
        return st;
    for (uint32_t i = 0; i < l->n_chunks; ++i) {
        const LinearChunk& ch = l->chunks[i];
        const size_t out_bytes = (size_t)ch.out_len * sizeof(float);
        BNN_Job job = {};
        job.operation = BNN_OP_GEMV_F32;
        job.matrix = ch.matrix;
        job.input.buffer = c->in_buf;
        job.input.type = BNN_TYPE_F32;
        job.output.buffer = c->out_buf;
        job.output.type = BNN_TYPE_F32;
        job.rows = 1;
        t0 = stats ? now_ns() : 0;
        st = accel_error(BNN_Execute(c->model->device, &job), "BNN_Execute");
        if (stats)
            c->stats.execute_ns += now_ns() - t0;
        if (st != BNNE_OK)
            return st;
        t0 = stats ? now_ns() : 0;
        st = accel_error(BNN_BufferRead(c->out_buf, 0, y + ch.out_off, out_bytes), "BNN_BufferRead");
        if (stats) {
            c->stats.transfer_ns += now_ns() - t0;
            c->stats.device_calls++;
            c->stats.bytes_read += out_bytes;
        }
        if (st != BNNE_OK)
            return st;
    }
    if (stats) {
        const uint64_t macs = (uint64_t)l->in * l->out;
        c->stats.logical_macs += macs;
        c->stats.executed_macs += macs;
    }
    return BNNE_OK;
}

BNNE_Status tensor_f32(const Gguf* g, const char* tensor, float** out, size_t* out_n) {
    if (!g || !tensor || !out || !out_n)
        return BNNE_EINVAL;
    const GgufTensor* t = gguf_find(g, tensor);
    if (!t || (t->type != kTypeF32 && t->type != kTypeF16))
        return error(BNNE_EFORMAT, "missing or invalid F32/F16 tensor '%s'", tensor);
    uint64_t count = 1;
    for (uint32_t d = 0; d < t->rank; ++d) {
        if (t->dims[d] == 0 || count > UINT64_MAX / t->dims[d])
            return error(BNNE_EFORMAT, "invalid shape for tensor '%s'", tensor);
        count *= t->dims[d];
    }
    if (count > SIZE_MAX / sizeof(float))
        return error(BNNE_ERANGE, "tensor '%s' is too large", tensor);
    auto* v = static_cast<float*>(alloc_array((size_t)count, sizeof(float)));
    if (!v)
        return error(BNNE_ENOMEM, "out of memory");
    const uint8_t* src = gguf_data(g, t);
    for (uint64_t i = 0; i < count; ++i) {
        if (t->type == kTypeF32) {
            const uint32_t bits = (uint32_t)src[4 * i] | ((uint32_t)src[4 * i + 1] << 8) |
                                  ((uint32_t)src[4 * i + 2] << 16) | ((uint32_t)src[4 * i + 3] << 24);
            std::memcpy(&v[i], &bits, 4);
        } else {
            v[i] = fp16_to_fp32(le16(src + 2 * i));
        }
        if (!std::isfinite(v[i])) {
            std::free(v);
            return error(BNNE_EFORMAT, "non-finite value in tensor '%s'", tensor);
        }
    }
    *out = v;
    *out_n = (size_t)count;
    return BNNE_OK;
}

}  // namespace bnne
