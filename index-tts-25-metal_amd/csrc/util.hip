// Weight layout conversion, prefix construction and beam bookkeeping kernels.
#include "kernels.h"

namespace itts {
namespace {

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return static_cast<uint16_t>((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// dst[o][i] = src[i][o] through a 32x33 LDS tile (gpt.cpp:24-33 does this on the host).
template <bool BF16>
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ src, void* __restrict__ dst, int in, int out) {
    __shared__ float tile[32][33];
    const int o0 = blockIdx.x * 32, i0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int i = i0 + r, o = o0 + tx;
        tile[r][tx] = (i < in && o < out) ? src[static_cast<size_t>(i) * out + o] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int o = o0 + r, i = i0 + tx;
        if (o < out && i < in) {
            const float v = tile[tx][r];
            if constexpr (BF16)
                static_cast<uint16_t*>(dst)[static_cast<size_t>(o) * in + i] = f32_to_bf16_rne(v);
            else
                static_cast<float*>(dst)[static_cast<size_t>(o) * in + i] = v;
        }
    }
}

template <bool BF16>
__global__ void convert_kernel(const float* __restrict__ src, void* __restrict__ dst, size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        if constexpr (BF16)
            static_cast<uint16_t*>(dst)[i] = f32_to_bf16_rne(src[i]);
        else
            static_cast<float*>(dst)[i] = src[i];
    }
}

// gpt.cpp:57-69: (text_emb[id] + text_pos[r]) + lang_emb[language]; final row mel_emb[8192] + mel_pos[0].
__global__ void text_rows_kernel(const float* text_emb, const float* text_pos, const float* lang_emb, const float* mel_emb,
                                 const float* mel_pos, const uint32_t* ids, int n_ids, uint32_t language, float* out) {
    const int r = blockIdx.x;
    for (int c = threadIdx.x; c < kWidth; c += blockDim.x) {
        float v;
        if (r < n_ids)
            v = (text_emb[static_cast<size_t>(ids[r]) * kWidth + c] + text_pos[static_cast<size_t>(r) * kWidth + c]) +
                lang_emb[static_cast<size_t>(language) * kWidth + c];
        else
            v = mel_emb[static_cast<size_t>(kMelStart) * kWidth + c] + mel_pos[c];
        out[static_cast<size_t>(r) * kWidth + c] = v;
    }
}

// mit2_linear_rows_f32_rowmajor (kernels.metal:1352-1374): acc = bias; acc += w*x in column
// order; then + emotion (gpt.cpp:53-54).
__global__ void speaker_row_kernel(const float* w, const float* b, const float* speaker, const float* emotion, float* out) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= kWidth) return;
    float acc = b[r];
    for (int c = 0; c < 192; ++c) acc = acc + w[static_cast<size_t>(r) * 192 + c] * speaker[c];
    out[r] = acc + emotion[r];
}

__global__ void gather_rows_kernel(const float* x, const uint32_t* src_rows, float* h) {
    const int b = blockIdx.x;
    for (int c = threadIdx.x; c < kWidth; c += blockDim.x)
        h[static_cast<size_t>(b) * kWidth + c] = x[static_cast<size_t>(src_rows[b]) * kWidth + c];
}

// Beam reorder: child c inherits parent[c]'s row owners (rows 0..n-1) and repetition set
// (plus its new token) and owns row n itself.  Parents are staged first so children may share them.
// Repetition sets of sequences 0..grid.y-1: exactly {1, 8192} (gpt_sampling.cpp:176).
__global__ void seen_reset_kernel(uint8_t* seen) {
    uint8_t* row = seen + static_cast<size_t>(blockIdx.y) * kMelVocab;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kMelVocab; i += gridDim.x * blockDim.x)
        row[i] = (i == 1 || i == kMelStart) ? 1 : 0;
}

// One sequence's prefill rows: slot 0, positions 0..rows-1, last row rows-1 (other
// sequences' last-row entries 0).
__global__ void prefill_rows_one_kernel(uint32_t* row_slot, uint32_t* row_pos, uint32_t* last_rows, uint32_t rows) {
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
        row_slot[r] = 0;
        row_pos[r] = r;
    }
    if (blockIdx.x == 0 && threadIdx.x < static_cast<unsigned>(kMaxBatch)) last_rows[threadIdx.x] = threadIdx.x == 0 ? rows - 1 : 0;
}

}  // namespace

hipError_t launch_seen_reset(uint8_t* seen, int nseq, hipStream_t s) {
    hipLaunchKernelGGL(seen_reset_kernel, dim3(8, nseq), dim3(256), 0, s, seen);
    return hipGetLastError();
}

hipError_t launch_prefill_rows_one(uint32_t* row_slot, uint32_t* row_pos, uint32_t* last_rows, uint32_t rows, hipStream_t s) {
    hipLaunchKernelGGL(prefill_rows_one_kernel, dim3(std::max(1u, std::min(4u, (rows + 255) / 256))), dim3(256), 0, s, row_slot,
                       row_pos, last_rows, rows);
    return hipGetLastError();
}

hipError_t launch_transpose(const float* src, void* dst, int in, int out, bool bf16, hipStream_t s) {
    const dim3 grid((out + 31) / 32, (in + 31) / 32);
    if (bf16)
        hipLaunchKernelGGL(transpose_kernel<true>, grid, dim3(256), 0, s, src, dst, in, out);
    else
        hipLaunchKernelGGL(transpose_kernel<false>, grid, dim3(256), 0, s, src, dst, in, out);
    return hipGetLastError();
}

hipError_t launch_convert(const float* src, void* dst, size_t n, bool bf16, hipStream_t s) {
    const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 4096));
    if (bf16)
        hipLaunchKernelGGL(convert_kernel<true>, dim3(blocks), dim3(256), 0, s, src, dst, n);
    else
        hipLaunchKernelGGL(convert_kernel<false>, dim3(blocks), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}

hipError_t launch_text_rows(const float* text_emb, const float* text_pos, const float* lang_emb, const float* mel_emb,
                            const float* mel_pos, const uint32_t* ids, int n_ids, uint32_t language, float* out,
                            hipStream_t s) {
    hipLaunchKernelGGL(text_rows_kernel, dim3(n_ids + 1), dim3(256), 0, s, text_emb, text_pos, lang_emb, mel_emb, mel_pos, ids,
                       n_ids, language, out);
    return hipGetLastError();
}

hipError_t launch_speaker_row(const float* w, const float* b, const float* speaker, const float* emotion, float* out,
                              hipStream_t s) {
    hipLaunchKernelGGL(speaker_row_kernel, dim3((kWidth + 255) / 256), dim3(256), 0, s, w, b, speaker, emotion, out);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float* x, const uint32_t* src_rows, float* h, int batch, hipStream_t s) {
    hipLaunchKernelGGL(gather_rows_kernel, dim3(batch), dim3(256), 0, s, x, src_rows, h);
    return hipGetLastError();
}

}  // namespace itts
