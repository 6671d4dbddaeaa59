// Per-wave timeline of the decode split kernel at the C2 headline shape
// (B = 1, 32768 keys, H 32 / Hkv 8 / head_dim 128, f16 K/V, fp32 query), or
// with the argument `gemma4` at Gemma 4's global-layer shape (H 16 / Hkv 1 /
// head_dim 512, attn_decode_mh_kernel), for measurement only: it is not part
// of libllmoxide_amd.so.
//
// It compiles the library's own kernel with LMX_DECODE_MARK defined, so that
// lane 0 of every wave stores s_memrealtime (100 MHz) at the kernel's phase
// marks, plus the wave's shader-clock cycles and its HW_ID / XCC_ID, then
// prints the phase distribution over the 1024 waves of one call and the
// per-XCD start / end.  The split plans are the library's for these shapes
// (headline: 2 units x 128 splits = 256 workgroups, 16 tiles a wave; gemma4:
// 256 splits of 8 tiles, every wave taking every tile).
//
// Build and run (repository root):
//   hipcc -O3 -std=c++17 --offload-arch=gfx950 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops -ffp-contract=fast -I include -I llmoxide_amd/csrc \
//     llmoxide_amd/timeline/decode_timeline.hip -o /tmp/decode_timeline
//   /tmp/decode_timeline            (or: /tmp/decode_timeline gemma4)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <string>
#include <vector>

__device__ unsigned long long g_tl[1024][8];
#define LMX_DECODE_MARK(i)                                                                      \
    do {                                                                                        \
        if ((threadIdx.x & 63) == 0) {                                                          \
            unsigned long long* r_ = g_tl[blockIdx.x * 4 + (threadIdx.x >> 6)];                 \
            r_[i] = __builtin_amdgcn_s_memrealtime();                                           \
            if ((i) == 0) r_[5] = __builtin_amdgcn_s_memtime();                                 \
            if ((i) == 4) {                                                                     \
                unsigned hw_, xcc_;                                                             \
                asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw_));               \
                asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_));             \
                r_[5] = __builtin_amdgcn_s_memtime() - r_[5];                                   \
                r_[6] = hw_;                                                                    \
                r_[7] = xcc_;                                                                   \
            }                                                                                   \
        }                                                                                       \
    } while (0)
#include "attn_decode.hpp"

#define CK(x)                                                                                   \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);          \
            return 1;                                                                           \
        }                                                                                       \
    } while (0)

int main(int argc, char** argv) {
    const bool g4 = argc > 1 && std::string(argv[1]) == "gemma4";
    const int H = g4 ? 16 : 32, Hkv = g4 ? 1 : 8, HD = g4 ? 512 : 128;
    constexpr int CTX = 32768, NL = 4;
    // the library's plans for these shapes
    const int P = g4 ? 256 : 128, N_YG = g4 ? 1 : 2, N_MAIN = 256;
    const int TPS = CTX / lmx::kTile / P;
    std::vector<float> hq(H * HD);
    unsigned s = 1;
    auto rnd = [&]() {
        s = s * 1664525u + 1013904223u;
        return ((s >> 8) & 0xffff) / 65536.f - 0.5f;
    };
    for (auto& x : hq) x = rnd();
    std::vector<_Float16> hk((size_t)CTX * Hkv * HD);
    for (auto& x : hk) x = (_Float16)rnd();
    float *q, *o, *po, *pml;
    CK(hipMalloc(&q, hq.size() * 4));
    CK(hipMalloc(&o, H * HD * 4));
    CK(hipMalloc(&po, (size_t)H * P * HD * 4));
    CK(hipMalloc(&pml, (size_t)H * P * 2 * 4));
    CK(hipMemcpy(q, hq.data(), hq.size() * 4, hipMemcpyHostToDevice));
    lmx::f16 *ks[NL], *vs[NL];  // rotated layer caches, as bench.py's headline
    for (int l = 0; l < NL; ++l) {
        CK(hipMalloc(&ks[l], hk.size() * 2));
        CK(hipMalloc(&vs[l], hk.size() * 2));
        CK(hipMemcpy(ks[l], hk.data(), hk.size() * 2, hipMemcpyHostToDevice));
        CK(hipMemcpy(vs[l], hk.data(), hk.size() * 2, hipMemcpyHostToDevice));
    }
    lmx::DecodeArgs a{};
    a.q = q;
    a.out = o;
    a.q_stride = HD;
    a.gate_stride = HD;
    a.part_o = po;
    a.part_ml = pml;
    a.H = H;
    a.Hkv = Hkv;
    a.G = H / Hkv;
    a.kv_dim = Hkv * HD;
    a.base_pos = CTX - 1;
    a.n_tokens = 1;
    a.P = P;
    a.tps = TPS;
    a.n_hblk = 1;  // both shapes: one head block a kv head
    a.n_q = 1;
    a.n_main = N_MAIN;
    a.n_yg = N_YG;
    a.m_parts = g4 ? 32 : 16;  // lanes a merged column: P / 8 rounded up to a power of two
    a.n_merge = (H * (HD / 4) * a.m_parts + lmx::kDecThreads - 1) / lmx::kDecThreads;
    a.c = (g4 ? 1.0f : 0.08838834764f) * 1.4426950408889634f;
    auto split = [&](int l) {
        a.k = ks[l];
        a.v = vs[l];
        if (g4)
            hipLaunchKernelGGL((lmx::attn_decode_mh_kernel<float, lmx::kModeLinear>), dim3(N_MAIN),
                               dim3(lmx::kDecThreads), 0, 0, a);
        else
            hipLaunchKernelGGL((lmx::attn_decode_kernel<float, 128, 4, 4, lmx::kModeLinear, false>), dim3(N_MAIN),
                               dim3(lmx::kDecThreads), 0, 0, a);
    };
    auto merge = [&]() {
        if (g4)
            hipLaunchKernelGGL((lmx::attn_merge_kernel<512, lmx::kModeLinear>), dim3(a.n_merge),
                               dim3(lmx::kDecThreads), 0, 0, a);
        else
            hipLaunchKernelGGL((lmx::attn_merge_kernel<128, lmx::kModeLinear>), dim3(a.n_merge),
                               dim3(lmx::kDecThreads), 0, 0, a);
    };
    for (int r = 0; r < 40; ++r) split(r % NL);
    CK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    constexpr int REP = 200;
    CK(hipEventRecord(e0));
    for (int r = 0; r < REP; ++r) {
        split(r % NL);
        merge();
    }
    CK(hipEventRecord(e1));
    CK(hipDeviceSynchronize());
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    std::printf("split + merge, back to back: %.2f us a call (%d calls over %d layer caches)\n", ms * 1e3 / REP,
                REP, NL);
    CK(hipEventRecord(e0));
    for (int r = 0; r < REP; ++r) split(r % NL);
    CK(hipEventRecord(e1));
    CK(hipDeviceSynchronize());
    CK(hipEventElapsedTime(&ms, e0, e1));
    std::printf("split kernel alone, back to back: %.2f us a call\n", ms * 1e3 / REP);

    // The timeline: one more call after the queue has drained.
    split(0);
    CK(hipDeviceSynchronize());
    static unsigned long long tl[1024][8];
    CK(hipMemcpyFromSymbol(tl, HIP_SYMBOL(g_tl), sizeof(tl)));
    constexpr int NW = N_MAIN * lmx::kWaves;
    unsigned long long t0 = ~0ull, t1 = 0;
    for (int i = 0; i < NW; ++i) {
        t0 = std::min(t0, tl[i][0]);
        t1 = std::max(t1, tl[i][4]);
    }
    auto us = [&](unsigned long long t) { return (double)(t - t0) / 100.0; };
    std::printf("one call: %.2f us from the first wave's start to the last wave's end\n", us(t1));
    std::vector<double> ph[7];
    double x_start[8], x_first[8] = {0}, x_end[8] = {0}, clk = 0;
    for (int x = 0; x < 8; ++x) x_start[x] = 1e30;
    for (int i = 0; i < NW; ++i) {
        for (int k = 0; k < 5; ++k) ph[k].push_back(us(tl[i][k]));
        ph[5].push_back((us(tl[i][3]) - us(tl[i][2])) / (TPS - 1));
        ph[6].push_back(us(tl[i][4]) - us(tl[i][3]));
        const int x = (int)(tl[i][7] & 7);
        x_start[x] = std::min(x_start[x], us(tl[i][0]));
        x_first[x] = std::max(x_first[x], us(tl[i][2]));
        x_end[x] = std::max(x_end[x], us(tl[i][4]));
        clk += (double)tl[i][5] / ((us(tl[i][4]) - us(tl[i][0])) * 1e-6) / NW;
    }
    const char* names[7] = {"wave start", "query loaded and converted", "first tile done", "last tile done",
                            "partials stored (wave end)", "per tile after the first", "epilogue (combine, stores)"};
    std::printf("%-28s %7s %7s %7s %7s %7s  (us; the first five from the call's first wave start)\n", "phase",
                "min", "p10", "median", "p90", "max");
    for (int k = 0; k < 7; ++k) {
        std::vector<double> v = ph[k];
        std::sort(v.begin(), v.end());
        std::printf("%-28s %7.2f %7.2f %7.2f %7.2f %7.2f\n", names[k], v[0], v[v.size() / 10], v[v.size() / 2],
                    v[v.size() * 9 / 10], v.back());
    }
    std::printf("shader clock (s_memtime cycles over each wave's span, averaged): %.2f GHz\n", clk / 1e9);
    for (int x = 0; x < 8; ++x)
        std::printf("XCD %d: first wave start %.2f, latest first tile %.2f, last wave end %.2f us\n", x, x_start[x],
                    x_first[x], x_end[x]);
    return 0;
}
