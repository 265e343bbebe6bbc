// route.hip -- router top-k and the drop-in pointer tables, on the GPU.
//
// The reference routes on the host side of every MoE layer
// (runtime/model_runner_v2.py:189-202 decode, :272-286 batch):
//     probs = softmax(logits.float()); topv, topi = topk(probs, k)
//     topv /= topv.sum(-1)                      (norm_topk_prob)
//     ids = topi.view(-1).tolist()              (host sync)
//     token-major pointer lists -> H2D tables   (moe_gateup / moe_down)
// Here both steps are kernels, so a decode step needs no host round trip and
// can be captured whole in a HIP graph:
//   router_topk_kernel    one wave per row: softmax over the row's n logits
//                         (max, exp, sum by wave reductions), then k rounds
//                         of a wave-wide argmax (ties: lower index first),
//                         then the renormalisation in rank order.
//   route_tables_kernel   the int64 pointer tables of moe_gateup_tab /
//                         moe_down_tab (entry m*2k + proj*k + e, and m*k + e)
//                         from the ids and the stacked expert weights.
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int kMaxN = 1024;   // experts per row
constexpr int kMaxK = 32;     // routed slots per row

// NPL logits per lane: element i*64 + lane of the row (mx::wave_topk).
template <int NPL>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int64_t ldl, int M,
                                                          int n, int k, int norm, int32_t* __restrict__ ids,
                                                          int64_t* __restrict__ ids64, float* __restrict__ w) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;   // the whole wave; no barriers below
    int id;
    float wt;
    mx::wave_topk<NPL>(logits + (int64_t)row * ldl, n, k, norm, id, wt);
    if (lane < k) {
        const int64_t o = (int64_t)row * k + lane;
        ids[o] = id;
        if (ids64) ids64[o] = id;
        w[o] = wt;
    }
}

struct TabArgs {
    const uint8_t* wp[3];   // gate, up, down packed data
    const uint8_t* ws[3];   // scales
    int64_t wp_stride[3];   // bytes between experts
    int64_t ws_stride[3];
    int64_t* gu_wp;         // (M, 2k): m*2k + proj*k + e
    int64_t* gu_ws;
    int64_t* dn_wp;         // (M, k): m*k + e
    int64_t* dn_ws;
    int n_experts;
};

__global__ __launch_bounds__(256) void route_tables_kernel(const int32_t* __restrict__ ids, int Mk, int k,
                                                           TabArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= Mk) return;
    const int m = i / k, e = i - m * k;
    int id = ids[i];
    id = id < 0 ? 0 : (id >= a.n_experts ? a.n_experts - 1 : id);   // memory safety only
    const int64_t g = (int64_t)m * 2 * k + e;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        a.gu_wp[g + p * k] = (int64_t)(a.wp[p] + id * a.wp_stride[p]);
        a.gu_ws[g + p * k] = (int64_t)(a.ws[p] + id * a.ws_stride[p]);
    }
    a.dn_wp[i] = (int64_t)(a.wp[2] + id * a.wp_stride[2]);
    a.dn_ws[i] = (int64_t)(a.ws[2] + id * a.ws_stride[2]);
}

}  // namespace

extern "C" int mxfp4_route_topk(const float* logits, int64_t ldl, int M, int n_experts, int k, int norm,
                                int32_t* ids, int64_t* ids64, float* w, void* stream) {
    MXH_REQUIRE(logits && ids && w, "route_topk: null pointer");
    MXH_REQUIRE(M > 0 && M < (1 << 26), "route_topk: M=%d", M);
    MXH_REQUIRE(n_experts > 0 && n_experts <= kMaxN, "route_topk: n_experts=%d (1..%d)", n_experts, kMaxN);
    MXH_REQUIRE(k > 0 && k <= kMaxK && k <= n_experts, "route_topk: k=%d (1..min(%d, n_experts))", k, kMaxK);
    MXH_REQUIRE(ldl >= n_experts, "route_topk: ldl=%lld < n_experts=%d", (long long)ldl, n_experts);
    const dim3 grid((M + 3) / 4), block(256);
    hipStream_t st = mxh::as_stream(stream);
    if (n_experts <= 128)
        hipLaunchKernelGGL(router_topk_kernel<2>, grid, block, 0, st, logits, ldl, M, n_experts, k, norm, ids, ids64, w);
    else if (n_experts <= 256)
        hipLaunchKernelGGL(router_topk_kernel<4>, grid, block, 0, st, logits, ldl, M, n_experts, k, norm, ids, ids64, w);
    else
        hipLaunchKernelGGL(router_topk_kernel<16>, grid, block, 0, st, logits, ldl, M, n_experts, k, norm, ids, ids64, w);
    return mxh::launch_status("route_topk");
}

extern "C" int mxfp4_route_tables(const int32_t* ids, int M, int k, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                  const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                  const uint8_t* down_ws, int n_experts, int H, int Mi, int64_t* gu_wp_tab,
                                  int64_t* gu_ws_tab, int64_t* dn_wp_tab, int64_t* dn_ws_tab, void* stream) {
    MXH_REQUIRE(ids && gate_wp && gate_ws && up_wp && up_ws && down_wp && down_ws, "route_tables: null pointer");
    MXH_REQUIRE(gu_wp_tab && gu_ws_tab && dn_wp_tab && dn_ws_tab, "route_tables: null table");
    MXH_REQUIRE(M > 0 && k > 0 && (int64_t)M * k < (1 << 28), "route_tables: M=%d k=%d", M, k);
    MXH_REQUIRE(n_experts > 0 && H > 0 && Mi > 0, "route_tables: n_experts=%d H=%d Mi=%d", n_experts, H, Mi);
    const int64_t hp = (H + 31) / 32 * 32, mp = (Mi + 31) / 32 * 32;   // Kp of gate/up and of down
    TabArgs a;
    a.wp[0] = gate_wp; a.ws[0] = gate_ws;
    a.wp[1] = up_wp;   a.ws[1] = up_ws;
    a.wp[2] = down_wp; a.ws[2] = down_ws;
    a.wp_stride[0] = a.wp_stride[1] = (int64_t)Mi * (hp / 2);
    a.ws_stride[0] = a.ws_stride[1] = (int64_t)Mi * (hp / 32);
    a.wp_stride[2] = (int64_t)H * (mp / 2);
    a.ws_stride[2] = (int64_t)H * (mp / 32);
    a.gu_wp = gu_wp_tab; a.gu_ws = gu_ws_tab;
    a.dn_wp = dn_wp_tab; a.dn_ws = dn_ws_tab;
    a.n_experts = n_experts;
    const int Mk = M * k;
    hipLaunchKernelGGL(route_tables_kernel, dim3((Mk + 255) / 256), dim3(256), 0, mxh::as_stream(stream), ids, Mk, k,
                       a);
    return mxh::launch_status("route_tables");
}
