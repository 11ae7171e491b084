// EnhancedCodec::decode (src/codec.cpp:57-72), the consumer of the GPT's semantic codes, on
// the MI355X: codes [T] -> features [2T][1024], time-major.
//
//   x      = out_project(codebook[codes])                       (codec.cpp:57-63; 8 -> 1024)
//   x      = LN(conv7(x))                                       (vocos_pass, codec.cpp:36-40; 1024 -> 384)
//   12 x:  x += gamma * pwconv2(GELU(pwconv1(LN(dwconv7(x))))) (codec.cpp:41-47; 384 -> 2048 -> 384)
//   y      = decoder.1(LN(x))                                   (codec.cpp:48; 384 -> 1024)
//   out    = conv3(nearest_x2(y))                               (codec.cpp:68-70; 1024 -> 1024 over 2T)
// LayerNorm eps 1e-6, biased variance (kernels.metal:618-669 with codec.cpp:28); GELU is the
// codec's erf form, erf from the Abramowitz-Stegun 7.1.26 polynomial (kernels.metal:3133-3137);
// "same" convolutions pad kernel/2 zeros on each side (kernels.metal:1397-1426, 1516-1541).
//
// Kernels:
//   * codec_lookup: one workgroup per code, the 8-wide codebook row times out_project.
//   * codec_gemm<EPI>: C = A W^T + bias on the FP32 matrix cores (v_mfma_f32_32x32x2f32),
//     64 x 64 tile per 256-thread workgroup, A with a row stride of its own.  Grids below
//     about 512 workgroups split K (partial sums, then codec_reduce adds them in split order
//     and applies the epilogue), since a decode of a few dozen codes gives only a handful of
//     output tiles.  A "same"
//     convolution of kernel k over time-major rows is this GEMM with K = k * Cin: row t of A
//     is the k consecutive input rows t .. t + k - 1 of the zero-padded input (contiguous
//     in memory, so A is the padded input read with row stride Cin), and the weights are
//     stored [Cout][k][Cin].  Epilogues: bias; bias + GELU; residual + gamma * (. + bias).
//   * codec_dwconv_ln: depthwise conv7 + LayerNorm of one 384-wide row per wave.
//   * codec_ln: LayerNorm of one 384-wide row per wave.
//   * codec_upsample: nearest x2 in time into the zero-padded input of the last conv.
// A decode of a given length is captured once as a HIP graph and replayed (about 60 launches,
// which bound short decodes); the padding rows are written by kernels, not memsets.
#include <type_traits>
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "itts_gpt.h"

namespace itts {
namespace {

constexpr int kCW = 1024;        // codec feature width
constexpr int kCH = 384;         // ConvNeXt width
constexpr int kCF = 2048;        // ConvNeXt hidden width
constexpr int kCBlocks = 12;
constexpr int kCK = 7;           // embed / depthwise kernel
constexpr int kUpK = 3;          // up conv kernel
constexpr int kCodebook = 8192;
constexpr int kCodeDim = 8;
constexpr int kMaxCodes = 5000;  // codec.cpp:58
constexpr float kCodecEps = 1e-6f;

typedef float floatx16 __attribute__((ext_vector_type(16)));

// 0.5 x (1 + erf(x / sqrt 2)), erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the form
// the reference's codec GELU evaluates.
__device__ __forceinline__ float codec_gelu(float x) {
    const float v = x * 0.7071067811865475f, a = fabsf(v), t = 1.0f / (1.0f + 0.3275911f * a);
    const float p = (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
    float erf = 1.0f - p * expf(-a * a);
    if (v < 0) erf = -erf;
    return 0.5f * x * (1.0f + erf);
}

// Row r of the embed conv's zero-padded input (T + 2 pad rows): rows pad .. pad + T - 1 are the
// projected codebook rows of the codes, the others zero.
__global__ __launch_bounds__(256) void codec_lookup_kernel(const uint32_t* codes, const float* cb, const float* w, const float* b,
                                                           float* out, int T, int pad) {
    const int r = blockIdx.x, tid = threadIdx.x;
    if (r < pad || r >= T + pad) {
#pragma unroll
        for (int i = 0; i < kCW / 256; ++i) out[static_cast<size_t>(r) * kCW + tid + 256 * i] = 0.0f;
        return;
    }
    const int t = r;
    __shared__ float e[kCodeDim];
    if (tid < kCodeDim) e[tid] = cb[static_cast<size_t>(codes[r - pad]) * kCodeDim + tid];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kCW / 256; ++i) {
        const int o = tid + 256 * i;
        const float* wr = w + static_cast<size_t>(o) * kCodeDim;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kCodeDim; ++j) acc = __builtin_fmaf(wr[j], e[j], acc);
        out[static_cast<size_t>(t) * kCW + o] = acc + b[o];
    }
}

enum CodecEpi : int { kEpiBias = 0, kEpiGelu = 1, kEpiScaleResid = 2 };

struct CodecGemm {
    const float* a;      // A rows, lda floats apart (rows may overlap: a convolution window)
    int lda;
    const float* w;      // [N][K]
    const float* bias;   // [N]
    const float* gamma;  // kEpiScaleResid: [N]
    float* c;            // [M][ldc]; kEpiScaleResid: read-modify-write residual
    int ldc;
    int M, N, K;
    float* ws;           // split-K partial sums [splits][M][N] (splits > 1)
    int kchunk;          // K per split (a multiple of GK)
};

constexpr int GM = 64, GN = 64, GK = 32, GP = 4;

__device__ __forceinline__ float codec_epilogue(int epi, float v, float gamma, const float* p) {
    if (epi == kEpiBias) return v;
    if (epi == kEpiGelu) return codec_gelu(v);
    return *p + v * gamma;  // codec.cpp:46: x + scale(h, gamma)
}

// One 64 x 64 tile of C over K range [z kchunk, (z + 1) kchunk): 2 x 2 waves of 32 x 32 MFMA
// tiles, 32 K per LDS stage with the next stage prefetched into registers.  PARTIAL: the raw
// sums go to ws[z]; otherwise bias and the epilogue are applied in place.
template <int EPI, bool PARTIAL>
__global__ __launch_bounds__(256) void codec_gemm_kernel(CodecGemm g) {
    __shared__ float As[GK][GM + GP];
    __shared__ float Bs[GK][GN + GP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
    const int k_begin = blockIdx.z * g.kchunk, k_end = min(g.K, k_begin + g.kchunk);
    const int lrow = tid >> 2, lk = (tid & 3) * 4;  // loader: K pieces lk and lk + 16 of one row
    const bool arow_ok = m0 + lrow < g.M;
    const float* arow = g.a + static_cast<size_t>(arow_ok ? m0 + lrow : 0) * g.lda + lk;
    const float* wrow = g.w + static_cast<size_t>(n0 + lrow) * g.K + lk;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 ra0 = zero, ra1 = zero, rb0, rb1;
    auto load = [&](int k0) {
        if (arow_ok) {
            ra0 = *reinterpret_cast<const float4*>(arow + k0);
            ra1 = *reinterpret_cast<const float4*>(arow + k0 + 16);
        }
        rb0 = *reinterpret_cast<const float4*>(wrow + k0);
        rb1 = *reinterpret_cast<const float4*>(wrow + k0 + 16);
    };
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    load(k_begin);
    for (int k0 = k_begin; k0 < k_end; k0 += GK) {
        As[lk + 0][lrow] = ra0.x;
        As[lk + 1][lrow] = ra0.y;
        As[lk + 2][lrow] = ra0.z;
        As[lk + 3][lrow] = ra0.w;
        As[lk + 16][lrow] = ra1.x;
        As[lk + 17][lrow] = ra1.y;
        As[lk + 18][lrow] = ra1.z;
        As[lk + 19][lrow] = ra1.w;
        Bs[lk + 0][lrow] = rb0.x;
        Bs[lk + 1][lrow] = rb0.y;
        Bs[lk + 2][lrow] = rb0.z;
        Bs[lk + 3][lrow] = rb0.w;
        Bs[lk + 16][lrow] = rb1.x;
        Bs[lk + 17][lrow] = rb1.y;
        Bs[lk + 18][lrow] = rb1.z;
        Bs[lk + 19][lrow] = rb1.w;
        __syncthreads();
        if (k0 + GK < k_end) load(k0 + GK);
#pragma unroll
        for (int kk = 0; kk < GK; kk += 2) {
            const float av = As[kk + (lane >> 5)][wm * 32 + (lane & 31)];
            const float bv = Bs[kk + (lane >> 5)][wn * 32 + (lane & 31)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    // D layout of v_mfma_f32_32x32x2f32: lane l, element i -> row 8(i/4) + 4(l/32) + i%4, col l%32.
    const int col = n0 + wn * 32 + (lane & 31);
    auto row_of = [&](int i) { return m0 + wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); };
    if constexpr (PARTIAL) {
        // Every destination formed before the first store: with one register pair reused for
        // each row's address, the compiler waited for each store to complete before forming
        // the next address.
        size_t dst[16];  // element offsets into ws (rows past M are formed, never stored to)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            dst[i] = (static_cast<size_t>(blockIdx.z) * g.M + row_of(i)) * g.N + col;
            asm volatile("" ::"v"(dst[i]));
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (row_of(i) < g.M) g.ws[dst[i]] = acc[i];
    } else {
        // Bias and gamma read once, every row's residual requested before the first store (rows
        // past M reread row M - 1, in bounds, and store nothing), and every value formed before
        // the first store.  Read per element behind the stores into C, which may alias them,
        // each was a memory round trip; and a use of a load inside a row's branch made the
        // compiler wait there for every access in flight, the earlier rows' stores included.
        const float bias = g.bias[col], gamma = EPI == kEpiScaleResid ? g.gamma[col] : 0.0f;
        float res[16], out[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            res[i] = EPI == kEpiScaleResid ? g.c[static_cast<size_t>(min(row_of(i), g.M - 1)) * g.ldc + col] : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            out[i] = codec_epilogue(EPI, acc[i] + bias, gamma, &res[i]);
            asm volatile("" ::"v"(out[i]));  // formed here, not sunk into the row's branch
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = row_of(i);
            if (row < g.M) g.c[static_cast<size_t>(row) * g.ldc + col] = out[i];
        }
    }
}

// Split-K: C = epilogue(sum over splits z = 0, 1, ... of ws[z] + bias), in split order, so
// the result does not depend on which split finished first.
template <int EPI>
__global__ __launch_bounds__(256) void codec_reduce_kernel(CodecGemm g, int splits) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x, total = static_cast<size_t>(g.M) * g.N;
    if (i >= total) return;
    const int row = static_cast<int>(i / g.N), col = static_cast<int>(i % g.N);
    float* p = g.c + static_cast<size_t>(row) * g.ldc + col;
    const float bias = g.bias[col], gamma = EPI == kEpiScaleResid ? g.gamma[col] : 0.0f;
    const float res = EPI == kEpiScaleResid ? *p : 0.0f;
    // every split's partial requested before the first add (SM >= splits; indices past the split
    // count reread the last split and are not added): a loop of dependent adds over loads issued
    // one at a time made each split a memory round trip
    auto sum = [&](auto sm) {
        constexpr int SM = decltype(sm)::value;
        float w[SM];
#pragma unroll
        for (int z = 0; z < SM; ++z) w[z] = g.ws[static_cast<size_t>(min(z, splits - 1)) * total + i];
        float s = 0.0f;
#pragma unroll
        for (int z = 0; z < SM; ++z)
            if (z < splits) s += w[z];
        return s;
    };
    const float s = splits <= 4 ? sum(std::integral_constant<int, 4>{})
                    : splits <= 8 ? sum(std::integral_constant<int, 8>{})
                    : splits <= 16 ? sum(std::integral_constant<int, 16>{})
                                   : sum(std::integral_constant<int, 32>{});
    *p = codec_epilogue(EPI, s + bias, gamma, &res);
}

// LayerNorm of a 384-wide row held as 6 values per lane (columns lane + 64 i): mean, then
// the biased variance of the centred values, eps 1e-6.
__device__ __forceinline__ void ln384(float (&v)[6], const float* gw, const float* gb, int lane) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 6; ++i) s += v[i];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    const float mean = s / float(kCH);
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const float d = v[i] - mean;
        q += d * d;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
    const float inv = 1.0f / sqrtf(q / float(kCH) + kCodecEps);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int c = lane + 64 * i;
        v[i] = (v[i] - mean) * inv * gw[c] + gb[c];
    }
}

// Depthwise conv7 (same padding) of row t, then LayerNorm: one wave per row, 4 rows per workgroup.
__global__ __launch_bounds__(256) void codec_dwconv_ln_kernel(const float* x, const float* dw, const float* db, const float* gw,
                                                              const float* gb, float* out, int T) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    // All 42 loads first (rows clamped into [0, T), taps outside it zeroed), so they are in
    // flight together instead of one tap's branch at a time.
    float xv[kCK][6];
#pragma unroll
    for (int k = 0; k < kCK; ++k) {
        const int src = t + k - kCK / 2;
        const int row = min(max(src, 0), T - 1);
#pragma unroll
        for (int i = 0; i < 6; ++i) xv[k][i] = x[static_cast<size_t>(row) * kCH + lane + 64 * i];
        if (src < 0 || src >= T) {
#pragma unroll
            for (int i = 0; i < 6; ++i) xv[k][i] = 0.0f;
        }
    }
    float v[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int c = lane + 64 * i;
        float acc = db[c];
#pragma unroll
        for (int k = 0; k < kCK; ++k) acc += xv[k][i] * dw[c * kCK + k];
        v[i] = acc;
    }
    ln384(v, gw, gb, lane);
#pragma unroll
    for (int i = 0; i < 6; ++i) out[static_cast<size_t>(t) * kCH + lane + 64 * i] = v[i];
}

// LayerNorm of each 384-wide row (in place allowed): one wave per row.
__global__ __launch_bounds__(256) void codec_ln_kernel(const float* x, const float* gw, const float* gb, float* out, int T) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    float v[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) v[i] = x[static_cast<size_t>(t) * kCH + lane + 64 * i];
    ln384(v, gw, gb, lane);
#pragma unroll
    for (int i = 0; i < 6; ++i) out[static_cast<size_t>(t) * kCH + lane + 64 * i] = v[i];
}

// upad row 1 + j = y row floor(j * 0.5) (the reference's scale in/out = 0.5) for j < 2T; rows
// 0 and 2T + 1 are the conv's zero padding.
__global__ __launch_bounds__(256) void codec_upsample_kernel(const float* y, float* upad, int T) {
    const int j = blockIdx.x;  // 0 .. 2T + 1
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (j > 0 && j <= 2 * T) v = reinterpret_cast<const float4*>(y + static_cast<size_t>((j - 1) / 2) * kCW)[threadIdx.x];
    reinterpret_cast<float4*>(upad + static_cast<size_t>(j) * kCW)[threadIdx.x] = v;  // 256 threads x float4 = 1024 floats
}

#define CODEC_CHECK(x)                                                                                                  \
    do {                                                                                                                \
        const hipError_t e_ = (x);                                                                                      \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(e_) + " in " #x); \
    } while (0)

template <typename T>
struct Buf {
    T* p = nullptr;
    size_t n = 0;
    Buf() = default;
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    ~Buf() {
        if (p) (void)hipFree(p);
    }
    bool ensure(size_t count) {  // true when the buffer moved
        if (count <= n) return false;
        if (p) CODEC_CHECK(hipFree(p));
        p = nullptr;
        n = 0;
        CODEC_CHECK(hipMalloc(&p, count * sizeof(T)));
        n = count;
        return true;
    }
    void upload(const std::vector<T>& v) {
        ensure(v.size());
        CODEC_CHECK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    }
};

// Splits of K that bring a small grid up to about 512 workgroups, each split at least 256 deep.
inline int codec_splits(int M, int N, int K) {
    const int tiles = (N / GN) * ((M + GM - 1) / GM);
    int s = std::max(1, std::min((512 + tiles - 1) / tiles, K / 256));
    return std::min(s, 32);
}

}  // namespace

// A named host tensor as the constructor takes it.
struct CodecTensor {
    const float* data;
    std::vector<int64_t> shape;
};

struct CodecEngine {
    hipStream_t stream = nullptr;
    hipEvent_t ev[2] = {};
    Buf<float> cb, op_w, op_b, emb_w, emb_b, n0_w, n0_b, fin_w, fin_b, dec_w, dec_b, up_w, up_b;
    struct Block {
        Buf<float> dw, db, lw, lb, w1, b1, w2, b2, gamma;
    } blk[kCBlocks];
    Buf<float> xpad, x, hn, f, y, upad, out, ws;
    Buf<uint32_t> dcodes;
    // Decodes of one length replay a captured graph (ITTS_CODEC_GRAPHS=0: eager launches).  A
    // buffer that moves bumps `generation`, and graphs captured before are dropped.
    bool use_graphs = true;
    uint64_t generation = 0, graph_generation = 0;
    std::unordered_map<int, hipGraphExec_t> graphs;

    static int used_splits(int M, int N, int K, int* kchunk) {
        const int splits = codec_splits(M, N, K);
        *kchunk = ((K + splits - 1) / splits + GK - 1) / GK * GK;
        return (K + *kchunk - 1) / *kchunk;
    }
    static size_t ws_need(int M, int N, int K) {
        int kc = 0;
        const int used = used_splits(M, N, K, &kc);
        return used > 1 ? static_cast<size_t>(used) * M * N : 0;
    }
    template <class B>
    void grow(B& b, size_t n) {
        if (b.ensure(n)) ++generation;
    }
    // Every buffer a decode of T codes touches, sized before anything is queued (and captured).
    void reserve(int T) {
        const size_t pad = kCK / 2;
        grow(dcodes, T);
        grow(xpad, (T + 2 * pad) * kCW);
        grow(x, static_cast<size_t>(T) * kCH);
        grow(hn, static_cast<size_t>(T) * kCH);
        grow(f, static_cast<size_t>(T) * kCF);
        grow(y, static_cast<size_t>(T) * kCW);
        grow(upad, static_cast<size_t>(2 * T + 2) * kCW);
        grow(out, static_cast<size_t>(2 * T) * kCW);
        size_t w = std::max({ws_need(T, kCH, kCK * kCW), ws_need(T, kCF, kCH), ws_need(T, kCH, kCF), ws_need(T, kCW, kCH),
                             ws_need(2 * T, kCW, kUpK * kCW)});
        grow(ws, std::max<size_t>(w, 1));
    }

    template <int EPI>
    void gemm(CodecGemm g) {
        if (g.N % GN || g.K % GK || g.M < 1) throw std::logic_error("codec GEMM shape");
        const int used = used_splits(g.M, g.N, g.K, &g.kchunk);
        const dim3 grid(g.N / GN, (g.M + GM - 1) / GM, used);
        if (used == 1) {
            hipLaunchKernelGGL((codec_gemm_kernel<EPI, false>), grid, dim3(256), 0, stream, g);
        } else {
            if (ws.n < static_cast<size_t>(used) * g.M * g.N) throw std::logic_error("codec split-K workspace not reserved");
            g.ws = ws.p;
            hipLaunchKernelGGL((codec_gemm_kernel<EPI, true>), grid, dim3(256), 0, stream, g);
            CODEC_CHECK(hipGetLastError());
            const size_t total = static_cast<size_t>(g.M) * g.N;
            hipLaunchKernelGGL(codec_reduce_kernel<EPI>, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, g, used);
        }
        CODEC_CHECK(hipGetLastError());
    }
    std::string last_error;

    ~CodecEngine() {
        drop_graphs();
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        if (stream) (void)hipStreamDestroy(stream);
    }

    // EnhancedCodec::EnhancedCodec (codec.cpp:5-20): the shapes the decode path reads, with the
    // reference's message.
    void create(const std::unordered_map<std::string, CodecTensor>& t) {
        auto get = [&](const std::string& name, std::vector<int64_t> shape) -> const float* {
            auto it = t.find(name);
            if (it == t.end()) throw std::runtime_error("Missing tensor: " + name);
            if (it->second.shape != shape) throw std::runtime_error("Unsupported 2.5 codec shape: " + name);
            return it->second.data;
        };
        auto vec = [](const float* p, size_t n) { return std::vector<float>(p, p + n); };
        // [Cout][Cin][k] -> [Cout][k][Cin]: a conv becomes a GEMM over k consecutive input rows
        auto conv_w = [](const float* p, int cout, int cin, int k) {
            std::vector<float> r(static_cast<size_t>(cout) * cin * k);
            for (int o = 0; o < cout; ++o)
                for (int i = 0; i < cin; ++i)
                    for (int j = 0; j < k; ++j)
                        r[(static_cast<size_t>(o) * k + j) * cin + i] = p[(static_cast<size_t>(o) * cin + i) * k + j];
            return r;
        };
        const std::string q = "codec.quantizer.quantizers.0", d = "codec.decoder.0";
        cb.upload(vec(get(q + ".codebook.weight", {kCodebook, kCodeDim}), static_cast<size_t>(kCodebook) * kCodeDim));
        op_w.upload(vec(get(q + ".out_project.weight", {kCW, kCodeDim}), static_cast<size_t>(kCW) * kCodeDim));
        op_b.upload(vec(get(q + ".out_project.bias", {kCW}), kCW));
        emb_w.upload(conv_w(get(d + ".embed.weight", {kCH, kCW, kCK}), kCH, kCW, kCK));
        emb_b.upload(vec(get(d + ".embed.bias", {kCH}), kCH));
        n0_w.upload(vec(get(d + ".norm.weight", {kCH}), kCH));
        n0_b.upload(vec(get(d + ".norm.bias", {kCH}), kCH));
        for (int i = 0; i < kCBlocks; ++i) {
            const std::string l = d + ".convnext." + std::to_string(i);
            Block& b = blk[i];
            b.dw.upload(vec(get(l + ".dwconv.weight", {kCH, 1, kCK}), static_cast<size_t>(kCH) * kCK));
            b.db.upload(vec(get(l + ".dwconv.bias", {kCH}), kCH));
            b.lw.upload(vec(get(l + ".norm.weight", {kCH}), kCH));
            b.lb.upload(vec(get(l + ".norm.bias", {kCH}), kCH));
            b.w1.upload(vec(get(l + ".pwconv1.weight", {kCF, kCH}), static_cast<size_t>(kCF) * kCH));
            b.b1.upload(vec(get(l + ".pwconv1.bias", {kCF}), kCF));
            b.w2.upload(vec(get(l + ".pwconv2.weight", {kCH, kCF}), static_cast<size_t>(kCH) * kCF));
            b.b2.upload(vec(get(l + ".pwconv2.bias", {kCH}), kCH));
            b.gamma.upload(vec(get(l + ".gamma", {kCH}), kCH));
        }
        fin_w.upload(vec(get(d + ".final_layer_norm.weight", {kCH}), kCH));
        fin_b.upload(vec(get(d + ".final_layer_norm.bias", {kCH}), kCH));
        dec_w.upload(vec(get("codec.decoder.1.weight", {kCW, kCH}), static_cast<size_t>(kCW) * kCH));
        dec_b.upload(vec(get("codec.decoder.1.bias", {kCW}), kCW));
        up_w.upload(conv_w(get("codec.up.weight", {kCW, kCW, kUpK}), kCW, kCW, kUpK));
        up_b.upload(vec(get("codec.up.bias", {kCW}), kCW));
        const char* env = std::getenv("ITTS_CODEC_GRAPHS");
        use_graphs = !(env && std::strcmp(env, "0") == 0);
        CODEC_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        for (auto& e : ev) CODEC_CHECK(hipEventCreate(&e));
    }

    void check_codes(const uint32_t* codes, uint32_t n) const {
        bool ok = n >= 1 && n <= static_cast<uint32_t>(kMaxCodes) && codes;
        for (uint32_t i = 0; ok && i < n; ++i) ok = codes[i] < static_cast<uint32_t>(kCodebook);
        if (!ok) throw std::invalid_argument("Codec expects 1..5000 code IDs in [0,8192)");
    }

    // The whole decode of T codes already in dcodes, queued on the stream (kernels only, into
    // buffers reserve(T) sized); result in out.
    void enqueue(int T) {
        const int pad = kCK / 2;
        hipStream_t s = stream;
        hipLaunchKernelGGL(codec_lookup_kernel, dim3(T + 2 * pad), dim3(256), 0, s, dcodes.p, cb.p, op_w.p, op_b.p, xpad.p, T, pad);
        CODEC_CHECK(hipGetLastError());
        const int rows4 = (T + 3) / 4;
        gemm<kEpiBias>({xpad.p, kCW, emb_w.p, emb_b.p, nullptr, x.p, kCH, T, kCH, kCK * kCW, nullptr, 0});
        hipLaunchKernelGGL(codec_ln_kernel, dim3(rows4), dim3(256), 0, s, x.p, n0_w.p, n0_b.p, x.p, T);
        CODEC_CHECK(hipGetLastError());
        for (int i = 0; i < kCBlocks; ++i) {
            const Block& b = blk[i];
            hipLaunchKernelGGL(codec_dwconv_ln_kernel, dim3(rows4), dim3(256), 0, s, x.p, b.dw.p, b.db.p, b.lw.p, b.lb.p, hn.p, T);
            CODEC_CHECK(hipGetLastError());
            gemm<kEpiGelu>({hn.p, kCH, b.w1.p, b.b1.p, nullptr, f.p, kCF, T, kCF, kCH, nullptr, 0});
            gemm<kEpiScaleResid>({f.p, kCF, b.w2.p, b.b2.p, b.gamma.p, x.p, kCH, T, kCH, kCF, nullptr, 0});
        }
        hipLaunchKernelGGL(codec_ln_kernel, dim3(rows4), dim3(256), 0, s, x.p, fin_w.p, fin_b.p, hn.p, T);
        CODEC_CHECK(hipGetLastError());
        gemm<kEpiBias>({hn.p, kCH, dec_w.p, dec_b.p, nullptr, y.p, kCW, T, kCW, kCH, nullptr, 0});
        hipLaunchKernelGGL(codec_upsample_kernel, dim3(2 * T + 2), dim3(256), 0, s, y.p, upad.p, T);
        CODEC_CHECK(hipGetLastError());
        gemm<kEpiBias>({upad.p, kCW, up_w.p, up_b.p, nullptr, out.p, kCW, 2 * T, kCW, kUpK * kCW, nullptr, 0});
    }

    void drop_graphs() {
        for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
        graphs.clear();
    }
    // One decode of T codes: a replay of its captured graph, or eager launches.
    void run(int T) {
        if (!use_graphs) {
            enqueue(T);
            return;
        }
        if (graph_generation != generation || graphs.size() >= 64) {
            drop_graphs();
            graph_generation = generation;
        }
        auto it = graphs.find(T);
        if (it == graphs.end()) {
            hipGraph_t g = nullptr;
            CODEC_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
            try {
                enqueue(T);
            } catch (...) {
                (void)hipStreamEndCapture(stream, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            CODEC_CHECK(hipStreamEndCapture(stream, &g));
            hipGraphExec_t exec = nullptr;
            const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            CODEC_CHECK(e);
            it = graphs.emplace(T, exec).first;
        }
        CODEC_CHECK(hipGraphLaunch(it->second, stream));
    }

    void decode(const uint32_t* codes, uint32_t n, float* host_out) {
        check_codes(codes, n);
        reserve(static_cast<int>(n));
        CODEC_CHECK(hipMemcpyAsync(dcodes.p, codes, n * 4, hipMemcpyHostToDevice, stream));
        run(static_cast<int>(n));
        CODEC_CHECK(hipMemcpyAsync(host_out, out.p, static_cast<size_t>(2) * n * kCW * 4, hipMemcpyDeviceToHost, stream));
        CODEC_CHECK(hipStreamSynchronize(stream));
    }

    // Mean duration of the device work of decode(n codes) over iters back-to-back runs, and its
    // FLOPs (the GEMMs; lookup, norms, depthwise convs and copies are < 0.5% of them).
    void bench(uint32_t n, uint32_t iters, float* avg_ms, double* flops) {
        if (!iters || n < 1 || n > static_cast<uint32_t>(kMaxCodes)) throw std::invalid_argument("Invalid codec benchmark request");
        std::vector<uint32_t> codes(n);
        for (uint32_t i = 0; i < n; ++i) codes[i] = (i * 2654435761u) % kCodebook;
        reserve(static_cast<int>(n));
        CODEC_CHECK(hipMemcpyAsync(dcodes.p, codes.data(), n * 4, hipMemcpyHostToDevice, stream));
        run(static_cast<int>(n));  // warm-up (and the graph's capture)
        CODEC_CHECK(hipEventRecord(ev[0], stream));
        for (uint32_t i = 0; i < iters; ++i) run(static_cast<int>(n));
        CODEC_CHECK(hipEventRecord(ev[1], stream));
        CODEC_CHECK(hipEventSynchronize(ev[1]));
        float ms = 0;
        CODEC_CHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        *avg_ms = ms / iters;
        const double T = n;
        *flops = 2.0 * T * kCH * kCK * kCW + kCBlocks * 2.0 * (2.0 * T * kCH * kCF) + 2.0 * T * kCW * kCH +
                 2.0 * (2 * T) * kCW * kUpK * kCW;
    }
};

}  // namespace itts

struct itts_codec {
    itts::CodecEngine e;
};

namespace {
thread_local std::string g_codec_create_error;

template <class F>
int codec_guarded(itts_codec* c, F&& f) {
    try {
        f();
        return ITTS_OK;
    } catch (const std::invalid_argument& e) {
        (c ? c->e.last_error : g_codec_create_error) = e.what();
        return ITTS_EINVAL;
    } catch (const std::runtime_error& e) {
        (c ? c->e.last_error : g_codec_create_error) = e.what();
        return ITTS_ERUNTIME;
    } catch (const std::exception& e) {
        (c ? c->e.last_error : g_codec_create_error) = e.what();
        return ITTS_ELOGIC;
    }
}

int codec_create(const std::unordered_map<std::string, itts::CodecTensor>& t, itts_codec** out) {
    if (!out) return ITTS_EINVAL;
    *out = nullptr;
    auto c = std::make_unique<itts_codec>();
    const int st = codec_guarded(nullptr, [&] { c->e.create(t); });
    if (st == ITTS_OK) *out = c.release();
    return st;
}
}  // namespace

extern "C" {

int itts_codec_create(const itts_tensor* tensors, int32_t count, itts_codec** out) {
    std::unordered_map<std::string, itts::CodecTensor> t;
    for (int32_t i = 0; tensors && i < count; ++i) {
        const itts_tensor& x = tensors[i];
        if (!x.name || !x.data || x.ndim < 0 || x.ndim > 4) {
            g_codec_create_error = "Invalid tensor table";
            return ITTS_EINVAL;
        }
        t[x.name] = {x.data, std::vector<int64_t>(x.shape, x.shape + x.ndim)};
    }
    return codec_create(t, out);
}

int itts_codec_create_from_bundle(const itts_bundle* b, itts_codec** out) {
    if (!b) {
        g_codec_create_error = "Invalid bundle";
        return ITTS_EINVAL;
    }
    std::unordered_map<std::string, itts::CodecTensor> t;
    const int32_t n = itts_bundle_count(b);
    for (int32_t i = 0; i < n; ++i) {
        itts_bundle_tensor bt{};
        if (itts_bundle_tensor_at(b, i, &bt) != ITTS_OK) continue;
        const std::string name = bt.name;
        if (name.rfind("codec.", 0) != 0 || bt.dtype != ITTS_DTYPE_F32) continue;
        t[name] = {static_cast<const float*>(bt.data), std::vector<int64_t>(bt.shape, bt.shape + bt.ndim)};
    }
    return codec_create(t, out);
}

void itts_codec_destroy(itts_codec* c) { delete c; }

const char* itts_codec_last_error(const itts_codec* c) { return c ? c->e.last_error.c_str() : g_codec_create_error.c_str(); }

int itts_codec_decode(itts_codec* c, const uint32_t* codes, uint32_t n, float* out) {
    if (!c) return ITTS_EINVAL;
    return codec_guarded(c, [&] {
        if (!out) throw std::invalid_argument("Codec expects 1..5000 code IDs in [0,8192)");
        c->e.decode(codes, n, out);
    });
}

int itts_codec_bench(itts_codec* c, uint32_t n, uint32_t iters, float* avg_ms, double* flops) {
    if (!c || !avg_ms || !flops) return ITTS_EINVAL;
    return codec_guarded(c, [&] { c->e.bench(n, iters, avg_ms, flops); });
}

}  // extern "C"
