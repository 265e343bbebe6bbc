// Compiled torch/pybind binding of the C ABI (include/mxfp4_hip.h).
//
// The module has two submodules with the surfaces of the reference's two
// compiled extensions:
//   linear  -- mxfp4_linear_ext  (src/ext/mxfp4_binding.cpp:21-50): forward
//   decode  -- mxfp4_decode_ext  (src/ext/mxfp4_decode_binding.cpp:44-243):
//              prequant, lin_pq, moe_gateup, moe_down, moe_combine,
//              moe_gateup_tab, moe_down_tab, attn_decode, kv_write
// Names, argument order and meaning, output shapes and dtypes, and the
// argument-check messages are the reference's.  Each op is a thin shim:
// checks, torch allocations on the input's device (caching allocator), then
// one or two C-ABI calls on torch's current HIP stream.  Host pointer
// tables go to the kernels as launch arguments (no device table, no
// blocking copy, where the reference builds an int64 device table per
// call).  Compiled by the host compiler (no device code here) and linked
// against libmxfp4_hip.so.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "mxfp4_hip.h"

namespace {

void require(bool cond, const char* msg) {
    if (!cond) throw std::runtime_error(msg);
}

// A non-zero C-ABI status becomes a RuntimeError with the library's message.
void check(int status, const char* what) {
    if (status != 0) {
        throw std::runtime_error(std::string(what) + " failed (status " + std::to_string(status) +
                                 "): " + mxfp4_last_error());
    }
}

void* stream_of(const torch::Tensor& t) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

const uint8_t* u8(const torch::Tensor& t) { return static_cast<const uint8_t*>(t.data_ptr()); }
uint8_t* u8m(const torch::Tensor& t) { return static_cast<uint8_t*>(t.data_ptr()); }
float* f32(const torch::Tensor& t) { return static_cast<float*>(t.data_ptr()); }

// Host pointer table of cuda uint8 tensors (the checks of
// src/ext/mxfp4_decode_binding.cpp:44-60), read straight from the Python
// list (or tuple): no std::vector<Tensor> of reference-counted copies, and the
// pointer array is a per-thread buffer reused from call to call (slot 0 = the
// packed data table, 1 = the scale table).  cols0 = size(1) of the first entry.
struct PtrTable {
    const uint8_t* const* p;
    int64_t cols0;
};

PtrTable ptr_table(const py::handle& seq, int slot, int64_t expect, const char* count_msg) {
    PyObject* fast = PySequence_Fast(seq.ptr(), "pointer table must be a list of tensors");
    if (fast == nullptr) throw py::error_already_set();
    const py::object keep = py::reinterpret_steal<py::object>(fast);
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(fast);
    require((int64_t)n == expect, count_msg);
    require(n > 0, "empty pointer table");
    thread_local std::vector<const uint8_t*> buf[2];
    std::vector<const uint8_t*>& p = buf[slot];
    p.resize((size_t)n);
    PyObject** items = PySequence_Fast_ITEMS(fast);
    int64_t cols0 = 0;
    for (Py_ssize_t i = 0; i < n; ++i) {
        require(THPVariable_Check(items[i]), "ptr table entries must be cuda uint8");
        const at::Tensor& t = THPVariable_Unpack(items[i]);
        require(t.is_cuda() && t.scalar_type() == torch::kUInt8, "ptr table entries must be cuda uint8");
        if (i == 0) cols0 = t.dim() >= 2 ? t.size(1) : 0;
        p[(size_t)i] = static_cast<const uint8_t*>(t.data_ptr());
    }
    return {p.data(), cols0};
}

int dtype_code(c10::ScalarType s) {
    return s == torch::kBFloat16 ? 0 : s == torch::kHalf ? 1 : 2;
}

// ---- mxfp4_linear_ext -------------------------------------------------------

// x (M,K) half|bf16, wp (N,Kp/2) u8, wsc (N,Kp/32) u8 -> f32 (M,N); activations
// are rounded to fp16 and MXFP4-quantized per 32-block (mxfp4_binding.cpp:21-45).
torch::Tensor forward(torch::Tensor x, torch::Tensor wp, torch::Tensor wsc) {
    require(x.is_cuda(), "x must be cuda");
    require(wp.is_cuda() && wsc.is_cuda(), "weights must be cuda");
    require(wp.scalar_type() == torch::kUInt8 && wsc.scalar_type() == torch::kUInt8,
            "weight tensors must be uint8");
    torch::Tensor xh = (x.scalar_type() == torch::kHalf || x.scalar_type() == torch::kBFloat16)
                           ? x : x.to(torch::kHalf);
    xh = xh.contiguous();
    wp = wp.contiguous();
    wsc = wsc.contiguous();
    const int M = (int)x.size(0), K = (int)x.size(1);
    const int N = (int)wp.size(0), Kp = (int)wp.size(1) * 2;
    auto y = torch::empty({M, N}, x.options().dtype(torch::kFloat32));
    if (M == 0 || N == 0) return y;
    const size_t wsb = mxfp4_linear_workspace_size(M, Kp);
    auto ws = torch::empty({(int64_t)wsb + 256}, x.options().dtype(torch::kUInt8));
    void* aligned = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(ws.data_ptr()) + 255) & ~uintptr_t(255));
    check(mxfp4_linear_forward(xh.data_ptr(), dtype_code(xh.scalar_type()), u8(wp), u8(wsc), f32(y),
                               M, N, K, Kp, aligned, wsb, stream_of(x)), "forward");
    return y;
}

// ---- mxfp4_decode_ext -------------------------------------------------------

// x (M,K) bf16 -> [xq (M,Kp/2) u8, xsc (M,Kp/32) u8], Kp = ceil32(K).
std::vector<torch::Tensor> prequant(torch::Tensor x) {
    require(x.is_cuda(), "x must be cuda");
    require(x.scalar_type() == torch::kBFloat16, "x must be bfloat16");
    x = x.contiguous();
    const int M = (int)x.size(0), K = (int)x.size(1);
    const int Kp = (K + 31) / 32 * 32;
    auto opts = x.options().dtype(torch::kUInt8);
    auto xq = torch::empty({M, Kp / 2}, opts);
    auto xsc = torch::empty({M, Kp / 32}, opts);
    if (M && Kp) {
        check(mxfp4_prequant(x.data_ptr(), K, M, K, Kp, u8m(xq), u8m(xsc), stream_of(x)), "prequant");
    }
    return {xq, xsc};
}

// Pre-quantized static linear -> f32 (M,N); Kp = 2*wp.size(1).
torch::Tensor lin_pq(torch::Tensor xq, torch::Tensor xsc, torch::Tensor wp, torch::Tensor wsc,
                     int64_t M_, int64_t N_, int64_t K_) {
    xq = xq.contiguous(); xsc = xsc.contiguous();
    wp = wp.contiguous(); wsc = wsc.contiguous();
    const int M = (int)M_, N = (int)N_, K = (int)K_;
    const int Kp = (int)wp.size(1) * 2;
    auto y = torch::empty({M, N}, xq.options().dtype(torch::kFloat32));
    check(mxfp4_lin_pq(u8(xq), u8(xsc), u8(wp), u8(wsc), f32(y), M, N, K, Kp, stream_of(xq)), "lin_pq");
    return y;
}

// Grouped gate+up over a token-major table of 2E*M weights -> f32 (M*E, 2N).
torch::Tensor moe_gateup(torch::Tensor xq, torch::Tensor xsc, const py::object& wps, const py::object& wscs,
                         int64_t E_, int64_t M_, int64_t N_, int64_t K_) {
    const int E = (int)E_, M = (int)M_, N = (int)N_, K = (int)K_;
    require((int64_t)py::len(wps) == 2 * E_ * M_, "wps must be 2E*M");
    require((int64_t)py::len(wscs) == 2 * E_ * M_, "wscs must be 2E*M");
    const PtrTable tw = ptr_table(wps, 0, 2 * E_ * M_, "wps must be 2E*M");
    const PtrTable ts = ptr_table(wscs, 1, 2 * E_ * M_, "wscs must be 2E*M");
    const int Kp = (int)tw.cols0 * 2;
    auto gu = torch::empty({(int64_t)M * E, 2 * N}, xq.options().dtype(torch::kFloat32));
    check(mxfp4_moe_gateup(u8(xq), u8(xsc), tw.p, ts.p, f32(gu), E, M, N, K, Kp, stream_of(xq)), "moe_gateup");
    return gu;
}

// Fused silu(gate)*up -> MXFP4 -> down over E*M weights -> f32 (M*E, N).
torch::Tensor moe_down(torch::Tensor gu, const py::object& wps, const py::object& wscs, int64_t E_, int64_t M_,
                       int64_t N_, int64_t K_) {
    const int E = (int)E_, M = (int)M_, N = (int)N_, K = (int)K_;
    require((int64_t)py::len(wps) == E_ * M_, "wps must be E*M");
    require(gu.size(0) == (int64_t)M * E && gu.size(1) == 2 * (int64_t)K, "gu (M*E,2K)");
    const PtrTable tw = ptr_table(wps, 0, E_ * M_, "wps must be E*M");
    const PtrTable ts = ptr_table(wscs, 1, E_ * M_, "wscs must be E*M");
    const int Kp = (int)tw.cols0 * 2;
    gu = gu.contiguous();
    auto yd = torch::empty({(int64_t)M * E, N}, gu.options());
    check(mxfp4_moe_down(f32(gu), tw.p, ts.p, f32(yd), E, M, N, K, Kp, stream_of(gu)), "moe_down");
    return yd;
}

// out[m,c] = sum_{e<min(E,8)} w[m,e]*yd[m*E+e,c] -> f32 (M,N); E = w.numel()/M.
torch::Tensor moe_combine(torch::Tensor yd, torch::Tensor w, int64_t M_) {
    yd = yd.contiguous(); w = w.contiguous();
    const int M = (int)M_;
    require(M > 0, "w (M,E)");
    const int E = (int)(w.numel() / M);
    const int N = (int)yd.size(1);
    require((int64_t)M * E == w.numel(), "w (M,E)");
    require(yd.size(0) == (int64_t)M * E, "yd (M*E,N)");
    auto out = torch::empty({M, N}, yd.options());
    check(mxfp4_moe_combine(f32(yd), N, f32(w), E, f32(out), M, N, stream_of(yd)), "moe_combine");
    return out;
}

// moe_gateup with device int64 pointer tables; Kp = 2*xq.size(1).
torch::Tensor moe_gateup_tab(torch::Tensor xq, torch::Tensor xsc, torch::Tensor wps_tab,
                             torch::Tensor wscs_tab, int64_t E_, int64_t M_, int64_t N_, int64_t K_) {
    const int E = (int)E_, M = (int)M_, N = (int)N_, K = (int)K_;
    const int Kp = (int)xq.size(1) * 2;
    auto gu = torch::empty({(int64_t)M * E, 2 * N}, xq.options().dtype(torch::kFloat32));
    check(mxfp4_moe_gateup_devtab(u8(xq), u8(xsc), static_cast<const int64_t*>(wps_tab.data_ptr()),
                                  static_cast<const int64_t*>(wscs_tab.data_ptr()), f32(gu), E, M, N, K,
                                  Kp, stream_of(xq)),
          "moe_gateup_tab");
    return gu;
}

// moe_down with device int64 pointer tables; Kp = ceil32(gu.size(1)/2).
torch::Tensor moe_down_tab(torch::Tensor gu, torch::Tensor wps_tab, torch::Tensor wscs_tab, int64_t E_,
                           int64_t M_, int64_t N_, int64_t K_) {
    const int E = (int)E_, M = (int)M_, N = (int)N_, K = (int)K_;
    const int Kp = (int)((gu.size(1) / 2 + 31) / 32 * 32);
    auto yd = torch::empty({(int64_t)M * E, N}, gu.options());
    check(mxfp4_moe_down_devtab(f32(gu), static_cast<const int64_t*>(wps_tab.data_ptr()),
                                static_cast<const int64_t*>(wscs_tab.data_ptr()), f32(yd), E, M, N, K, Kp,
                                stream_of(gu)),
          "moe_down_tab");
    return yd;
}

void check_kv(const torch::Tensor& kvk, const torch::Tensor& kvv, const torch::Tensor& dpos) {
    require(kvk.scalar_type() == torch::kUInt8 && kvv.scalar_type() == torch::kUInt8 && kvk.dim() == 3 &&
                kvv.sizes() == kvk.sizes(),
            "kvk/kvv must be uint8 (max_pos,Hkv,D) tensors of one shape");
    require(kvk.is_contiguous() && kvv.is_contiguous(), "kvk/kvv must be contiguous");
    require(dpos.scalar_type() == torch::kInt32 && dpos.is_cuda(), "dpos must be a cuda int32 tensor");
}

// Decode attention over one layer's E4M3 KV cache -> f32 (M,Hq,D).  q (M,Hq,D)
// bf16 (roped); dpos (1,) int32 on the device, token m attends to 0..dpos+m;
// sc (M,Hq,max_pos) f32 receives the raw scores (mxfp4_decode_binding.cpp:213-230).
torch::Tensor attn_decode(torch::Tensor q, torch::Tensor kvk, torch::Tensor kvv, torch::Tensor dpos,
                          torch::Tensor sc, int64_t M_) {
    require(q.dim() == 3 && q.scalar_type() == torch::kBFloat16 && q.is_cuda(),
            "q must be a cuda bf16 (M,Hq,D) tensor");
    q = q.contiguous();
    const int M = (int)M_;
    check_kv(kvk, kvv, dpos);
    const int Hq = (int)q.size(1), D = (int)q.size(2);
    const int max_pos = (int)kvk.size(0), Hkv = (int)kvk.size(1);
    require(q.size(0) >= M, "q has fewer than M rows");
    require(sc.scalar_type() == torch::kFloat32 && sc.is_contiguous() && sc.numel() >= (int64_t)M * Hq * max_pos,
            "sc must be a contiguous f32 buffer of M*Hq*max_pos elements");
    auto o = torch::empty({M, Hq, D}, q.options().dtype(torch::kFloat32));
    const size_t wsb = mxfp4_attn_decode_workspace_size(M, Hq, max_pos);
    auto ws = torch::empty({(int64_t)wsb}, q.options().dtype(torch::kUInt8));
    check(mxfp4_attn_decode(q.data_ptr(), u8(kvk), u8(kvv), static_cast<const int*>(dpos.data_ptr()), f32(sc),
                            f32(o), M, Hq, Hkv, D, max_pos, ws.data_ptr(), wsb, stream_of(q)),
          "attn_decode");
    return o;
}

// k/v (M,Hkv,D) bf16 -> E4M3 bytes at rows dpos+m of kvk/kvv (max_pos,Hkv,D)
// u8, in place (mxfp4_decode_binding.cpp:161-173).
void kv_write(torch::Tensor k, torch::Tensor v, torch::Tensor kvk, torch::Tensor kvv, torch::Tensor dpos,
              int64_t M_) {
    require(k.scalar_type() == torch::kBFloat16 && v.scalar_type() == torch::kBFloat16 && k.is_cuda() &&
                v.is_cuda(),
            "k/v must be cuda bf16");
    k = k.contiguous(); v = v.contiguous();
    const int M = (int)M_;
    check_kv(kvk, kvv, dpos);
    const int max_pos = (int)kvk.size(0), Hkv = (int)kvk.size(1), D = (int)kvk.size(2);
    require(k.numel() >= (int64_t)M * Hkv * D && v.numel() >= (int64_t)M * Hkv * D,
            "k/v have fewer than M*Hkv*D elements");
    check(mxfp4_kv_write(k.data_ptr(), v.data_ptr(), u8m(kvk), u8m(kvv), static_cast<const int*>(dpos.data_ptr()),
                         M, Hkv, D, max_pos, stream_of(k)),
          "kv_write");
}

}  // namespace

PYBIND11_MODULE(mxfp4_ext, m) {
    m.doc() = "Compiled torch binding of libmxfp4_hip (gfx950)";
    auto lin = m.def_submodule("linear", "mxfp4_linear_ext surface");
    lin.attr("__name__") = "mxfp4_linear_ext";
    lin.def("forward", &forward, "x (M,K) half|bf16 -> fp16 round -> MXFP4 -> f32 (M,N)");
    auto dec = m.def_submodule("decode", "mxfp4_decode_ext surface");
    dec.attr("__name__") = "mxfp4_decode_ext";
    dec.def("prequant", &prequant, "bf16 (M,K) -> [xq (M,Kp/2) u8, xsc (M,Kp/32) u8]");
    dec.def("lin_pq", &lin_pq, "prequantized static MXFP4 linear -> f32 (M,N)");
    dec.def("moe_gateup", &moe_gateup, "grouped gate+up (2E*M weights) -> f32 (M*E,2N)");
    dec.def("moe_down", &moe_down, "fused silu(gate)*up, MXFP4, down -> f32 (M*E,N)");
    dec.def("moe_combine", &moe_combine, "out[m,c] = sum_e w[m,e]*yd[m*E+e,c]");
    dec.def("moe_gateup_tab", &moe_gateup_tab, "grouped gate+up from device pointer tables");
    dec.def("moe_down_tab", &moe_down_tab, "fused silu-down from device pointer tables");
    dec.def("attn_decode", &attn_decode, "decode attention over an E4M3 KV cache -> f32 (M,Hq,D)");
    dec.def("kv_write", &kv_write, "E4M3 KV write of M tokens at rows dpos+m");
}
