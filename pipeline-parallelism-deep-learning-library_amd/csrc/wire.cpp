// The "LNGL" wire format of stage boundaries (crates/core/src/lib.rs:298-412), and the two
// device-buffer ends of a boundary: send_tensor's download + encode_wire and recv_tensor's
// decode_wire + upload (crates/pipeline/src/lib.rs:71-98), each as one direct copy between the
// device tensor and the caller's wire buffer, with no intermediate host tensor.
//
// Layout: "LNGL", u32 version 1, u32 dtype tag, u32 ndim (<= 8), ndim u32 extents, then the
// row-major payload; all little-endian. Errors follow the reference: a malformed message, a
// rank above 8 or an undecodable tag is Wire; an extent above u32::MAX or a byte count that
// overflows is Shape.
#include <cstring>

#include "lg_internal.h"

namespace lg {
namespace {

constexpr uint32_t WIRE_VERSION = 1;
constexpr uint32_t WIRE_MAX_NDIM = 8;
constexpr uint8_t WIRE_MAGIC[4] = {'L', 'N', 'G', 'L'};

struct WireErr {
    lg_core_error code;
    const char* message;
};

[[noreturn]] void wfail(lg_core_error code, const char* msg) { throw WireErr{code, msg}; }

uint64_t size_of(uint32_t tag) {
    switch (tag) {
        case LG_DTYPE_F32:
            return 4;
        case LG_DTYPE_F16:
        case LG_DTYPE_BF16:
            return 2;
    }
    wfail(LG_CORE_WIRE, "unknown dtype tag");
}

void put_u32(uint8_t* p, uint32_t v) {
    p[0] = static_cast<uint8_t>(v);
    p[1] = static_cast<uint8_t>(v >> 8);
    p[2] = static_cast<uint8_t>(v >> 16);
    p[3] = static_cast<uint8_t>(v >> 24);
}

uint32_t get_u32(const uint8_t* p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
           (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
}

// checked_nbytes (crates/core/src/lib.rs:396-405).
uint64_t checked_nbytes(uint32_t tag, const uint64_t* shape, uint32_t rank) {
    const uint64_t size = size_of(tag);
    uint64_t numel = 1;
    for (uint32_t d = 0; d < rank; ++d) {
        if (shape[d] > 0xffffffffull) wfail(LG_CORE_SHAPE, "extent above u32::MAX");
        if (shape[d] != 0 && numel > UINT64_MAX / shape[d]) wfail(LG_CORE_SHAPE, "element count overflows");
        numel *= shape[d];
    }
    if (numel > UINT64_MAX / size) wfail(LG_CORE_SHAPE, "byte count overflows");
    return numel * size;
}

// write_header (crates/core/src/lib.rs:337-357): (header length, payload bytes).
uint64_t write_header(uint32_t tag, const uint64_t* shape, uint32_t rank, uint8_t* out,
                      uint64_t* nbytes) {
    if (rank > WIRE_MAX_NDIM) wfail(LG_CORE_WIRE, "more than 8 extents");
    *nbytes = checked_nbytes(tag, shape, rank);
    std::memcpy(out, WIRE_MAGIC, 4);
    put_u32(out + 4, WIRE_VERSION);
    put_u32(out + 8, tag);
    put_u32(out + 12, rank);
    for (uint32_t d = 0; d < rank; ++d) put_u32(out + 16 + 4 * d, static_cast<uint32_t>(shape[d]));
    return 16 + 4ull * rank;
}

// parse_wire_header (crates/core/src/lib.rs:361-389).
uint64_t parse_header(const uint8_t* bytes, uint64_t len, uint32_t* tag, uint64_t* shape,
                      uint32_t* rank) {
    if (bytes == nullptr && len != 0) wfail(LG_CORE_WIRE, "null message");
    if (len < 16 || std::memcmp(bytes, WIRE_MAGIC, 4) != 0) wfail(LG_CORE_WIRE, "bad magic or short message");
    if (get_u32(bytes + 4) != WIRE_VERSION) wfail(LG_CORE_WIRE, "unsupported wire version");
    const uint32_t t = get_u32(bytes + 8);
    const uint64_t size = size_of(t);
    const uint32_t ndim = get_u32(bytes + 12);
    if (ndim > WIRE_MAX_NDIM) wfail(LG_CORE_WIRE, "more than 8 extents");
    const uint64_t header = 16 + 4ull * ndim;
    if (len < header) wfail(LG_CORE_WIRE, "message ends inside the extents");
    uint64_t numel = 1;
    for (uint32_t d = 0; d < ndim; ++d) {
        const uint64_t e = get_u32(bytes + 16 + 4 * d);
        if (e != 0 && numel > UINT64_MAX / e) wfail(LG_CORE_SHAPE, "element count overflows");
        numel *= e;
    }
    if (numel > UINT64_MAX / size) wfail(LG_CORE_SHAPE, "byte count overflows");
    if (len - header != numel * size) wfail(LG_CORE_WIRE, "payload length does not match the shape");
    *tag = t;
    *rank = ndim;
    for (uint32_t d = 0; d < ndim; ++d) shape[d] = get_u32(bytes + 16 + 4 * d);
    return header;
}

// strides == row_major_strides(shape) (crates/core/src/lib.rs:275-283); the running product
// wraps as the reference's does in release builds.
bool row_major_tensor(const lg_tensor* t) {
    if (t->nstrides != t->rank || t->rank > LG_MAX_RANK) return false;
    uint64_t stride = 1;
    for (uint32_t d = t->rank; d-- > 0;) {
        if (t->strides[d] != stride) return false;
        stride *= t->shape[d];
    }
    return true;
}

// Row-major contiguous at offset 0 (packed_layout, crates/cpu/src/lib.rs:735-747).
bool packed_tensor(const lg_tensor* t) { return t->offset == 0 && row_major_tensor(t); }

template <typename F>
lg_core_error wire_op(F&& body) {
    try {
        body();
        clear_last_error();
        return LG_CORE_OK;
    } catch (const WireErr& e) {
        set_last_error(e.message);
        return e.code;
    } catch (const Failure& f) {
        set_last_error(f.message);
        return LG_CORE_UNSUPPORTED_DEVICE;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return LG_CORE_UNSUPPORTED_DEVICE;
    } catch (...) {
        set_last_error("internal error: unknown exception");
        return LG_CORE_UNSUPPORTED_DEVICE;
    }
}

}  // namespace
}  // namespace lg

using namespace lg;

extern "C" {

lg_core_error lg_wire_write_header(uint32_t dtype, const uint64_t* shape, uint32_t rank,
                                   uint8_t out[LG_WIRE_HEADER_MAX], uint64_t* len) {
    return wire_op([&] {
        if (out == nullptr || len == nullptr || (shape == nullptr && rank != 0)) {
            wfail(LG_CORE_SHAPE, "null argument");
        }
        uint8_t tmp[LG_WIRE_HEADER_MAX];
        uint64_t nbytes = 0;
        const uint64_t n = write_header(dtype, shape, rank, tmp, &nbytes);
        std::memcpy(out, tmp, n);  // `out` changes only on success, and only its first n bytes
        *len = n;
    });
}

lg_core_error lg_wire_parse_header(const uint8_t* bytes, uint64_t len, uint32_t* dtype,
                                   uint64_t shape[8], uint32_t* rank, uint64_t* payload_offset) {
    return wire_op([&] {
        if (dtype == nullptr || shape == nullptr || rank == nullptr || payload_offset == nullptr) {
            wfail(LG_CORE_SHAPE, "null argument");
        }
        uint32_t t = 0, r = 0;
        uint64_t s[WIRE_MAX_NDIM] = {0};
        const uint64_t off = parse_header(bytes, len, &t, s, &r);
        *dtype = t;
        *rank = r;
        for (uint32_t d = 0; d < r; ++d) shape[d] = s[d];
        *payload_offset = off;
    });
}

lg_core_error lg_wire_encode(uint32_t dtype, const uint64_t* shape, uint32_t rank,
                             const void* payload, uint64_t payload_len, uint8_t* out,
                             uint64_t out_cap, uint64_t* written) {
    return wire_op([&] {
        if (written == nullptr || (shape == nullptr && rank != 0)) wfail(LG_CORE_SHAPE, "null argument");
        uint8_t head[LG_WIRE_HEADER_MAX];
        uint64_t nbytes = 0;
        const uint64_t h = write_header(dtype, shape, rank, head, &nbytes);
        if (payload_len != nbytes) wfail(LG_CORE_WIRE, "payload length does not match the shape");
        if (h > UINT64_MAX - nbytes) wfail(LG_CORE_SHAPE, "message length overflows");
        if (out == nullptr || out_cap < h + nbytes) wfail(LG_CORE_SHAPE, "output buffer too small");
        std::memcpy(out, head, h);
        if (nbytes) std::memcpy(out + h, payload, nbytes);
        *written = h + nbytes;
    });
}

lg_core_error lg_wire_encode_tensor(lg_ctx* ctx, const lg_tensor* t, uint8_t* out,
                                    uint64_t out_cap, uint64_t* written) {
    return wire_op([&] {
        if (t == nullptr || written == nullptr) wfail(LG_CORE_SHAPE, "null argument");
        const uint64_t size = size_of(t->dtype);  // a Tensor's dtype is a DType: decode it first
        if (t->rank > LG_MAX_RANK) wfail(LG_CORE_SHAPE, "rank above LG_MAX_RANK");
        // Backend::download (crates/cpu/src/lib.rs:183-194): row-major strides at any offset,
        // then the byte range [offset*size, offset*size + numel*size) inside the storage.
        if (!row_major_tensor(t)) wfail(LG_CORE_UNSUPPORTED_LAYOUT, "tensor is not row-major");
        uint64_t count = 1;
        for (uint32_t d = 0; d < t->rank; ++d) {
            if (t->shape[d] != 0 && count > UINT64_MAX / t->shape[d]) wfail(LG_CORE_SHAPE, "element count overflows");
            count *= t->shape[d];
        }
        if (t->offset > UINT64_MAX / size) wfail(LG_CORE_SHAPE, "offset overflows");
        if (count > UINT64_MAX / size) wfail(LG_CORE_SHAPE, "byte count overflows");
        const uint64_t start = t->offset * size, len = count * size;
        if (start > UINT64_MAX - len) wfail(LG_CORE_SHAPE, "byte range overflows");
        if (start + len > t->bytes) wfail(LG_CORE_SHAPE, "tensor reaches past its storage");
        // encode_wire (crates/core/src/lib.rs:309-322).
        uint8_t head[LG_WIRE_HEADER_MAX];
        uint64_t nbytes = 0;
        const uint64_t h = write_header(t->dtype, t->shape, t->rank, head, &nbytes);
        if (h > UINT64_MAX - nbytes) wfail(LG_CORE_SHAPE, "message length overflows");
        if (out == nullptr || out_cap < h + nbytes) wfail(LG_CORE_SHAPE, "output buffer too small");
        if (ctx == nullptr) wfail(LG_CORE_UNSUPPORTED_DEVICE, "null context");
        set_device(ctx);
        // After every earlier call on the context stream, like Backend::download.
        if (nbytes) {
            const uint8_t* src = static_cast<const uint8_t*>(t->base) + start;
            check_hip(hipMemcpyAsync(out + h, src, nbytes, hipMemcpyDeviceToHost, ctx->stream),
                      "hipMemcpyAsync");
        }
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        std::memcpy(out, head, h);
        *written = h + nbytes;
    });
}

lg_core_error lg_wire_decode_into(lg_ctx* ctx, const uint8_t* bytes, uint64_t len,
                                  const lg_tensor* t) {
    return wire_op([&] {
        if (t == nullptr) wfail(LG_CORE_SHAPE, "null argument");
        uint32_t tag = 0, rank = 0;
        uint64_t shape[WIRE_MAX_NDIM] = {0};
        const uint64_t h = parse_header(bytes, len, &tag, shape, &rank);
        if (tag != t->dtype) wfail(LG_CORE_DTYPE, "message dtype differs from the tensor's");
        if (rank != t->rank) wfail(LG_CORE_SHAPE, "message shape differs from the tensor's");
        for (uint32_t d = 0; d < rank; ++d) {
            if (shape[d] != t->shape[d]) wfail(LG_CORE_SHAPE, "message shape differs from the tensor's");
        }
        if (!packed_tensor(t)) wfail(LG_CORE_UNSUPPORTED_LAYOUT, "tensor is not row-major at offset 0");
        const uint64_t nbytes = len - h;
        if (nbytes > t->bytes) wfail(LG_CORE_SHAPE, "tensor reaches past its storage");
        if (ctx == nullptr) wfail(LG_CORE_UNSUPPORTED_DEVICE, "null context");
        set_device(ctx);
        if (nbytes) {
            check_hip(hipMemcpyAsync(t->base, bytes + h, nbytes, hipMemcpyHostToDevice, ctx->stream),
                      "hipMemcpyAsync");
        }
        // The bytes may be reused as soon as this returns (Backend::upload_into's rule).
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

}  // extern "C"
