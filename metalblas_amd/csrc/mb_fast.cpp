// Compiled fast path of the Python API for call signatures that are already planned.
//
// The first call of a signature (dtype, sizes, strides, pointer alignment classes, device,
// autotuner switch) goes through the Python layer (metalblas_amd/dispatch.py), which checks
// the operands, plans and tunes the product and registers the finished descriptor here.  Later
// calls of `matmul` (2-D, or an N-D A folded onto a 2-D B) and `bmm` with the same signature
// allocate the output, patch the descriptor's pointers and call mb_gemm without re-entering
// Python: about 3 us of host time per call less on small products.  Anything this path does
// not recognise (CPU tensors, conj views, views without a unit stride, empty shapes, a
// signature not seen yet) returns None, and the caller takes the Python path, which keeps
// every check and error of the reference's API.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <array>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <unordered_map>

#include "../../include/metalblas_amd.h"

namespace {

constexpr int kKeyLen = 19;
using Key = std::array<int64_t, kKeyLen>;

struct KeyHash {
    size_t operator()(const Key &k) const noexcept {
        uint64_t h = 1469598103934665603ull;
        for (int64_t v : k) {
            h ^= (uint64_t)v;
            h *= 1099511628211ull;
        }
        return (size_t)h;
    }
};

struct Entry {
    mb_gemm_desc desc;
    int64_t ws_bytes;
};

constexpr size_t kCap = 4096;
std::unordered_map<Key, Entry, KeyHash> g_cache;

// split-K scratch per (device, stream): the kernels of one stream run in order, so one call's
// scratch is free again for the next call on that stream
struct WsKey {
    int dev;
    void *stream;
    bool operator==(const WsKey &o) const { return dev == o.dev && stream == o.stream; }
};
struct WsHash {
    size_t operator()(const WsKey &k) const noexcept { return std::hash<void *>()(k.stream) ^ (size_t)k.dev; }
};
std::unordered_map<WsKey, at::Tensor, WsHash> g_ws;
constexpr int64_t kWsKeep = int64_t(64) << 20;

int dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return MB_DTYPE_F32;
        case at::kHalf: return MB_DTYPE_F16;
        case at::kBFloat16: return MB_DTYPE_BF16;
        case at::kComplexFloat: return MB_DTYPE_C64;
        case at::kComplexHalf: return MB_DTYPE_C32;
        case at::kChar: return MB_DTYPE_I8;
        case at::kByte: return MB_DTYPE_U8;
        case at::kShort: return MB_DTYPE_I16;
        case at::kInt: return MB_DTYPE_I32;
        case at::kLong: return MB_DTYPE_I64;
        default: return -1;
    }
}

bool autotune_on() {
    const char *v = std::getenv("METALBLAS_AUTOTUNE");
    return !(v && v[0] == '0' && v[1] == '\0');
}

// (row stride, column stride, batch stride) of a 2-D or 3-D tensor, as the descriptor takes them
void strides3(const at::Tensor &t, int64_t &rs, int64_t &cs, int64_t &bs) {
    if (t.dim() == 3) {
        bs = t.stride(0);
        rs = t.stride(1);
        cs = t.stride(2);
    } else {
        bs = 0;
        rs = t.stride(0);
        cs = t.stride(1);
    }
}

// the layouts the Python layer passes through unchanged (metalblas/dispatch.py:23-30): a unit
// stride along one of the last two dims and a leading stride covering the other
bool unit_lead(const at::Tensor &t, int64_t rows, int64_t cols) {
    const int64_t s0 = t.stride(t.dim() - 2), s1 = t.stride(t.dim() - 1);
    return (s1 == 1 && s0 >= cols) || (s0 == 1 && s1 >= rows);
}

Key make_key(int dt, int64_t batch, int64_t M, int64_t N, int64_t K, const at::Tensor &a, const at::Tensor &b,
             const at::Tensor &c) {
    Key k;
    int64_t rs, cs, bs;
    k[0] = dt;
    k[1] = batch;
    k[2] = M;
    k[3] = N;
    k[4] = K;
    strides3(a, rs, cs, bs);
    k[5] = rs; k[6] = cs; k[7] = bs;
    k[8] = (int64_t)((uintptr_t)a.data_ptr() & 255);
    strides3(b, rs, cs, bs);
    k[9] = rs; k[10] = cs; k[11] = bs;
    k[12] = (int64_t)((uintptr_t)b.data_ptr() & 255);
    strides3(c, rs, cs, bs);
    k[13] = rs; k[14] = cs; k[15] = bs;
    k[16] = (int64_t)((uintptr_t)c.data_ptr() & 255);
    k[17] = c.get_device();
    k[18] = autotune_on() ? 1 : 0;
    return k;
}

// operands the fast path takes: CUDA (HIP) tensors on the current device, one dtype, no conj
// view, a supported dtype, the reference's in-place layouts
bool operands_ok(const at::Tensor &a, const at::Tensor &b, int &dt) {
    if (!a.is_cuda() || !b.is_cuda() || a.scalar_type() != b.scalar_type() || a.is_conj() || b.is_conj())
        return false;
    if (a.get_device() != b.get_device() || a.get_device() != (int)c10::hip::current_device()) return false;
    dt = dtype_code(a.scalar_type());
    return dt >= 0;
}

// queue the cached plan for (a, b) -> c, or return false when the signature is not cached
bool launch_cached(int dt, int64_t batch, int64_t M, int64_t N, int64_t K, const at::Tensor &a, const at::Tensor &b,
                   const at::Tensor &c) {
    const auto it = g_cache.find(make_key(dt, batch, M, N, K, a, b, c));
    if (it == g_cache.end()) return false;
    mb_gemm_desc d = it->second.desc;
    d.a.ptr = a.data_ptr();
    d.b.ptr = b.data_ptr();
    d.c.ptr = c.data_ptr();
    const int dev = c.get_device();
    hipStream_t st = c10::hip::getCurrentHIPStream(dev).stream();
    at::Tensor once;   // a per-call workspace: freed after the launch is queued
    const int64_t ws_bytes = it->second.ws_bytes;
    if (ws_bytes > 0) {
        // under HIP graph capture the per-call tensor comes from the graph's private pool, which
        // the graph holds for its replays; the kept one could be replaced and freed meanwhile
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
        if (ws_bytes <= kWsKeep && cap == hipStreamCaptureStatusNone) {
            at::Tensor &ws = g_ws[WsKey{dev, (void *)st}];
            if (!ws.defined() || ws.numel() < ws_bytes)
                ws = at::empty({std::max<int64_t>(ws_bytes, int64_t(1) << 20)}, c.options().dtype(at::kByte));
            d.workspace = ws.data_ptr();
        } else {
            once = at::empty({ws_bytes}, c.options().dtype(at::kByte));
            d.workspace = once.data_ptr();
        }
        d.workspace_bytes = ws_bytes;
    }
    const int status = mb_gemm(&d, (void *)st);
    if (status != MB_OK) throw std::runtime_error(std::string("metalblas_amd: ") + mb_strerror(status));
    return true;
}

py::object fast_matmul(const at::Tensor &a, const at::Tensor &b) {
    int dt;
    if (b.dim() != 2 || a.dim() < 2 || !operands_ok(a, b, dt)) return py::none();
    const int64_t K = a.size(-1), N = b.size(1);
    if (b.size(0) != K || K == 0 || N == 0 || !unit_lead(b, K, N)) return py::none();
    if (a.dim() == 2) {
        const int64_t M = a.size(0);
        if (M == 0 || !unit_lead(a, M, K)) return py::none();
        at::Tensor c = at::empty({M, N}, a.options());
        if (!launch_cached(dt, 1, M, N, K, a, b, c)) return py::none();
        return py::cast(c);
    }
    // (..., M, K) @ (K, N) with A contiguous: one 2-D product over the folded rows
    if (!a.is_contiguous() || a.numel() == 0) return py::none();
    const at::Tensor a2 = a.view({-1, K});
    const int64_t rows = a2.size(0);
    at::Tensor c = at::empty({rows, N}, a.options());
    if (!launch_cached(dt, 1, rows, N, K, a2, b, c)) return py::none();
    std::vector<int64_t> shape(a.sizes().begin(), a.sizes().end());
    shape.back() = N;
    return py::cast(c.view(shape));
}

py::object fast_bmm(const at::Tensor &a, const at::Tensor &b) {
    int dt;
    if (a.dim() != 3 || b.dim() != 3 || !operands_ok(a, b, dt)) return py::none();
    const int64_t B = a.size(0), M = a.size(1), K = a.size(2), N = b.size(2);
    if (b.size(0) != B || b.size(1) != K || B == 0 || M == 0 || N == 0 || K == 0) return py::none();
    if (!unit_lead(a, M, K) || !unit_lead(b, K, N)) return py::none();
    at::Tensor c = at::empty({B, M, N}, a.options());
    if (!launch_cached(dt, B, M, N, K, a, b, c)) return py::none();
    return py::cast(c);
}

// Python registers the descriptor it planned (and tuned) for a product with no epilogue, no
// conj flag and no tile / backend / swizzle request; a, b, c are the tensors it launched.
void register_plan(const at::Tensor &a, const at::Tensor &b, const at::Tensor &c, py::bytes desc, int64_t ws_bytes) {
    const std::string s = desc;
    if (s.size() != sizeof(mb_gemm_desc)) throw std::runtime_error("metalblas_amd: descriptor size mismatch");
    Entry e;
    std::memcpy(&e.desc, s.data(), sizeof(mb_gemm_desc));
    e.ws_bytes = ws_bytes;
    if (g_cache.size() >= kCap) g_cache.clear();
    g_cache[make_key(e.desc.dtype, e.desc.batch, e.desc.M, e.desc.N, e.desc.K, a, b, c)] = e;
}

void clear() { g_cache.clear(); }

size_t size() { return g_cache.size(); }

}  // namespace

PYBIND11_MODULE(_fast, m) {
    m.doc() = "metalblas_amd compiled fast path for planned call signatures";
    m.def("matmul", &fast_matmul, "a @ b for a planned signature, else None");
    m.def("bmm", &fast_bmm, "batched a @ b for a planned signature, else None");
    m.def("register", &register_plan, "cache the descriptor Python planned for (a, b, c)");
    m.def("clear", &clear);
    m.def("size", &size);
}
