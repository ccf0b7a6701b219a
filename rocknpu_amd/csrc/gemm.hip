// Kernel (c): prefill W8A8 GEMM on CDNA4 int8 MFMA with the rescale fused.
//
// C_i32[m,n] = sum_k A8[m,k] * W8[n,k]   (exact; |C| <= 127^2 * K < 2^31)
// out[m,n]   = (f32(C) * a_scale[m]) * w_scale[n]
// which is the reference's M-tile product and rescale_i32_row
// (crates/rocknpu-capi/src/lib.rs:692-709, :1868-1884; NPU program
// crates/rocknpu-regcmd/src/int8.rs:112-205). Both operands are K-contiguous
// int8 rows; K is a multiple of 64 (rows are zero-padded, which is exact).
//
// Tiling: a workgroup computes a BM x BN tile with WM x WN waves; each wave
// owns a (BM/WM) x (BN/WN) sub-tile of 16x16 MFMA fragments
// (v_mfma_i32_16x16x64_i8: lane l supplies row l%16 and the 16 bytes of
// k-slot l/16 for both operands; it receives rows 4*(l/16)+i, column l%16).
// K advances in 64-byte slabs through double-buffered LDS with an XOR swizzle
// on the 16-byte chunk index so fragment reads are bank-conflict free.
#include "common.h"

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;

__device__ __forceinline__ int swz(int r, int kc) { return r * kBK + ((kc ^ ((r >> 1) & 3)) << 4); }

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void gemm_w8a8_kernel(
    const int8_t* __restrict__ a8, int64_t lda, const int8_t* __restrict__ w8, int64_t ldw,
    const float* __restrict__ a_scales, const float* __restrict__ w_scales, int m, int n, int k,
    float* __restrict__ out, int64_t ldo, int32_t* __restrict__ out_i32, int64_t ldo_i32) {
    constexpr int T = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int A_CHUNKS = BM * kBK / 16, B_CHUNKS = BN * kBK / 16;
    constexpr int A_PER = (A_CHUNKS + T - 1) / T, B_PER = (B_CHUNKS + T - 1) / T;
    static_assert(FM >= 1 && FN >= 1, "wave tile must hold at least one 16x16 fragment");
    __shared__ __align__(16) int8_t As[2][BM * kBK];
    __shared__ __align__(16) int8_t Bs[2][BN * kBK];

    const int tiles_n = (n + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    uint4 ra[A_PER], rb[B_PER];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * T;
            const int r = c >> 2, kc = c & 3;
            const int gr = m0 + r;
            ra[i] = (c < A_CHUNKS && gr < m)
                        ? *reinterpret_cast<const uint4*>(a8 + gr * lda + kt * kBK + kc * 16)
                        : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * T;
            const int r = c >> 2, kc = c & 3;
            const int gr = n0 + r;
            rb[i] = (c < B_CHUNKS && gr < n)
                        ? *reinterpret_cast<const uint4*>(w8 + gr * ldw + kt * kBK + kc * 16)
                        : make_uint4(0, 0, 0, 0);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * T;
            if (c < A_CHUNKS) *reinterpret_cast<uint4*>(&As[buf][swz(c >> 2, c & 3)]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * T;
            if (c < B_CHUNKS) *reinterpret_cast<uint4*>(&Bs[buf][swz(c >> 2, c & 3)]) = rb[i];
        }
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int KT = k / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        v4i af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
            af[i] = *reinterpret_cast<const v4i*>(&As[cur][swz(wm * TM + i * 16 + (lane & 15), lane >> 4)]);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            bf[j] = *reinterpret_cast<const v4i*>(&Bs[cur][swz(wn * TN + j * 16 + (lane & 15), lane >> 4)]);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * TN + j * 16 + (lane & 15);
            if (col >= n) continue;
            const float ws = w_scales[col];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + e;
                if (row >= m) continue;
                const int v = acc[i][j][e];
                const float t = static_cast<float>(v) * a_scales[row];
                out[row * ldo + col] = t * ws;
                if (out_i32) out_i32[row * ldo_i32 + col] = v;
            }
        }
}

template <int BM, int BN, int WM, int WN>
int launch_cfg(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
               const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
               int64_t ldoi, hipStream_t stream) {
    const int64_t tiles = static_cast<int64_t>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    gemm_w8a8_kernel<BM, BN, WM, WN><<<dim3(static_cast<unsigned>(tiles)), dim3(WM * WN * 64), 0, stream>>>(
        a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace

int launch_gemm_w8a8(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                     const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                     int64_t ldoi, hipStream_t stream) {
    if (m <= 16) return launch_cfg<16, 64, 1, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    if (m <= 32) return launch_cfg<32, 64, 1, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    if (m <= 256) return launch_cfg<64, 64, 2, 2>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    return launch_cfg<128, 128, 2, 2>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
}

}  // namespace rk
