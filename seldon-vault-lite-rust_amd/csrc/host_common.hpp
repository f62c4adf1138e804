// Host-side helpers shared by the text runtime (runtime.cpp) and the vision
// runtime (vision.cpp): the thread-local error message, status macros,
// growable device buffers, and weight-inventory validation / decoding in the
// manner of src/model/weights.rs:125-189 and src/binary/safetensors.rs:69-110.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "../../include/svl_hip.h"

struct svl_ctx {
    int device;
};

namespace svl {

inline thread_local std::string g_err;

inline svl_status fail(svl_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return st;
}

#define HIP_TRY(expr)                                                                       \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return fail(SVL_DEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define ST_TRY(expr)                    \
    do {                                \
        svl_status s_ = (expr);         \
        if (s_ != SVL_OK) return s_;    \
    } while (0)

// src/tensor/owned.rs MAX_TENSOR_ELEMENTS, text.rs:34 MAX_ACTIVATION_ELEMENTS.
constexpr int64_t MAX_ACTIVATION_ELEMENTS = int64_t(1) << 28;
constexpr int64_t MAX_TENSOR_ELEMENTS = int64_t(1) << 30;

template <class T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;
    hipError_t ensure(size_t count) {
        if (count <= n) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        hipError_t e = hipMalloc((void **)&p, std::max<size_t>(count, 1) * sizeof(T));
        if (e == hipSuccess) n = count;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
};

using ShapeList = std::vector<std::pair<std::string, std::vector<int64_t>>>;
using TensorIndex = std::map<std::string, const svl_tensor_view *>;

// Inventory check of a weight set (weights.rs:130-165, vision.rs:556-594):
// a tensor under one of `prefixes` that the shape list does not name is
// unexpected (CORRUPT), a named tensor that is absent or mis-shaped is
// CORRUPT, and the per-tensor and total element caps give LIMIT.
inline svl_status check_inventory(const svl_tensor_view *tensors, size_t n_tensors,
                                  const ShapeList &shapes,
                                  std::initializer_list<const char *> prefixes, const char *kind,
                                  int64_t max_total, TensorIndex &by_name) {
    by_name.clear();
    for (size_t i = 0; i < n_tensors; ++i) {
        if (!tensors[i].name) return fail(SVL_USAGE, "tensor %zu has no name", i);
        by_name[tensors[i].name] = &tensors[i];
    }
    std::map<std::string, size_t> expected;
    for (size_t i = 0; i < shapes.size(); ++i) expected[shapes[i].first] = i;
    for (auto &kv : by_name) {
        bool ours = false;
        for (const char *p : prefixes) ours = ours || kv.first.rfind(p, 0) == 0;
        if (ours && !expected.count(kv.first))
            return fail(SVL_CORRUPT, "unexpected %s tensor %s in the weight file", kind,
                        kv.first.c_str());
    }
    int64_t parameters = 0;
    for (auto &sh : shapes) {
        auto it = by_name.find(sh.first);
        if (it == by_name.end())
            return fail(SVL_CORRUPT, "%s weight %s is missing from the Safetensors file", kind,
                        sh.first.c_str());
        const svl_tensor_view *t = it->second;
        bool same = t->ndim == (int32_t)sh.second.size();
        for (size_t d = 0; same && d < sh.second.size(); ++d) same = t->shape[d] == sh.second[d];
        if (!same)
            return fail(SVL_CORRUPT, "%s weight %s has an unexpected shape", kind, sh.first.c_str());
        int64_t numel = 1;
        for (int64_t d : sh.second) numel *= d;
        if (numel > MAX_TENSOR_ELEMENTS)
            return fail(SVL_LIMIT, "tensor %s has %lld elements, above the cap", sh.first.c_str(),
                        (long long)numel);
        parameters += numel;
        if (parameters > max_total)
            return fail(SVL_LIMIT, "%s weights exceed the %lld-element cap", kind,
                        (long long)max_total);
        if (!t->data) return fail(SVL_USAGE, "tensor %s has no data", sh.first.c_str());
    }
    return SVL_OK;
}

// TensorEntry::to_f32 (safetensors.rs:69-110): F32 little-endian or BF16
// widened exactly (bf16.rs:13-15, bits << 16), each after the payload length
// check of the reference (safetensors.rs:79-88, bf16.rs:40-51). numel is at
// most MAX_TENSOR_ELEMENTS, so the byte counts cannot overflow. Non-finite
// values are rejected like Tensor::validate_finite (owned.rs:126-135).
inline svl_status widen_f32(const svl_tensor_view &t, int64_t numel, float *out) {
    if (t.dtype == SVL_F32) {
        const uint64_t expected = (uint64_t)numel * 4;
        if (t.nbytes != expected)
            return fail(SVL_CORRUPT, "tensor %s has %llu bytes, expected %llu for %lld F32 values",
                        t.name, (unsigned long long)t.nbytes, (unsigned long long)expected,
                        (long long)numel);
        if (numel > 0) std::memcpy(out, t.data, (size_t)numel * 4);
    } else if (t.dtype == SVL_BF16) {
        const uint64_t expected = (uint64_t)numel * 2;
        if (t.nbytes != expected)
            return fail(SVL_CORRUPT, "BF16 length mismatch: expected %llu bytes for %lld values, "
                        "got %llu", (unsigned long long)expected, (long long)numel,
                        (unsigned long long)t.nbytes);
        const uint16_t *b = (const uint16_t *)t.data;
        for (int64_t i = 0; i < numel; ++i) {
            const uint32_t bits = (uint32_t)b[i] << 16;
            std::memcpy(&out[(size_t)i], &bits, 4);
        }
    } else {
        return fail(SVL_UNSUPPORTED, "tensor %s has an unsupported dtype", t.name);
    }
    return SVL_OK;
}

inline svl_status decode_f32(const svl_tensor_view &t, int64_t numel, std::vector<float> &out) {
    out.resize((size_t)numel);
    if (svl_status st = widen_f32(t, numel, out.data())) return st;
    for (int64_t i = 0; i < numel; ++i)
        if (!std::isfinite(out[(size_t)i]))
            return fail(SVL_INTERNAL, "non-finite tensor value at index %lld of %s",
                        (long long)i, t.name);
    return SVL_OK;
}

inline svl_status decode_named(const TensorIndex &by_name, const std::string &name,
                               std::vector<float> &out) {
    auto it = by_name.find(name);
    if (it == by_name.end()) return fail(SVL_INTERNAL, "decoded tensor %s is missing", name.c_str());
    const svl_tensor_view *t = it->second;
    int64_t numel = 1;
    for (int d = 0; d < t->ndim; ++d) numel *= t->shape[d];
    return decode_f32(*t, numel, out);
}

// Copies a host array into a new device allocation recorded in `owned`.
inline svl_status upload_owned(std::vector<float *> &owned, const float *host, size_t count,
                               float **dst) {
    float *d = nullptr;
    HIP_TRY(hipMalloc((void **)&d, std::max<size_t>(count, 1) * sizeof(float)));
    owned.push_back(d);
    HIP_TRY(hipMemcpy(d, host, count * sizeof(float), hipMemcpyHostToDevice));
    *dst = d;
    return SVL_OK;
}

// Gate and up projections [I, H] interleaved in 32-row blocks
// [g 0..31, u 0..31, g 32..63, ...], padded to I_pad rows each, for the
// GeGLU epilogue of the gate/up GEMM.
inline std::vector<float> interleave_gate_up(const std::vector<float> &gate,
                                             const std::vector<float> &up, int64_t I,
                                             int64_t I_pad, int64_t H) {
    std::vector<float> gu((size_t)(2 * I_pad * H), 0.f);
    for (int64_t j = 0; j < I; ++j) {
        const int64_t blk = j / 32, off = j % 32;
        std::copy(gate.begin() + j * H, gate.begin() + (j + 1) * H,
                  gu.begin() + (64 * blk + off) * H);
        std::copy(up.begin() + j * H, up.begin() + (j + 1) * H,
                  gu.begin() + (64 * blk + 32 + off) * H);
    }
    return gu;
}

// Device handle of a text model, for the image prompt glue: runs a text
// batch with soft-token features already in HBM (d_feats, rows indexed by
// featmap) and returns the normalized embeddings on the host.
svl_status text_forward_with_device_features(svl_text_model *m, const uint32_t *ids,
                                             const int64_t *offsets, int32_t batch,
                                             const int32_t *featmap, const float *d_feats,
                                             float *out_normalized);
int text_device(const svl_text_model *m);
int64_t text_hidden_size(const svl_text_model *m);
int64_t text_embedding_dim(const svl_text_model *m);
int64_t text_pad_token(const svl_text_model *m);

}  // namespace svl
