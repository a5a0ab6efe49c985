// Layout and reduction kernels of the matmul path:
//  * tensor permute (cl_kernels/permute.cl:11-50): a batched 2-D transpose through LDS
//    when the permutation swaps the last two axes (the [0,2,1] / [1,0] forms that
//    BmmOp.Backward and the Python Linear use), else a generic <=10-D gather;
//  * column sums (cs/cl_kernels/linear.cl:149-168 linear_bias_backward and
//    cs/cl_kernels/reduce_sum_axis.cl:3-24 reduce_sum_axis): each output is summed over
//    the reduced axis in ascending order from +0.0f, exactly as the reference kernels do,
//    so these results are bit-identical to the reference's.
#include "migemm_internal.h"

namespace migemm {
namespace {

constexpr int MAXD = 10;

// FastDiv / make_fastdiv / fast_div: migemm_internal.h.
struct PermuteArgs {
    const float *src;
    float *dst;
    int64_t total;
    int ndim;
    int narrow;  // total < 2^31: every index and offset fits 32 bits
    int64_t dst_dims[MAXD];
    int64_t src_stride_of_dst_axis[MAXD];  // stride in src of the axis placed at dst axis i
    FastDiv div[MAXD];                     // dst_dims as invariant divisors (narrow only)
};

// dst[t] = src[offset of t's destination coordinates], coordinates from the last axis
// (permute.cl:2-8,11-50), on the canonical form built by launch_permute. Element t is a
// group of VW floats (VW = 4 when the innermost destination axis is contiguous in the source
// too); total, dims and strides are in those units. Tensors under 2^31 elements unpack t
// with 32-bit invariant divisions: with one 64-bit division and remainder per axis per
// element the kernel was bound by integer arithmetic, not by memory.
template <int VW>
__global__ void __launch_bounds__(256) permute_gather_kernel(PermuteArgs a) {
    typedef float vec __attribute__((ext_vector_type(VW)));
    const vec *src = reinterpret_cast<const vec *>(a.src);
    vec *dst = reinterpret_cast<vec *>(a.dst);
    if (a.narrow) {
        const uint32_t total = (uint32_t)a.total;
        const uint32_t step = gridDim.x * blockDim.x;
        for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += step) {
            uint32_t rem = t;
            uint32_t off = 0;
            for (int i = a.ndim - 1; i >= 0; --i) {
                const uint32_t q = fast_div(rem, a.div[i]);
                off += (rem - q * a.div[i].d) * (uint32_t)a.src_stride_of_dst_axis[i];
                rem = q;
            }
            dst[t] = src[off];
        }
        return;
    }
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < a.total; t += step) {
        int64_t rem = t;
        int64_t off = 0;
        for (int i = a.ndim - 1; i >= 0; --i) {
            const int64_t d = a.dst_dims[i];
            const int64_t c = rem % d;
            rem /= d;
            off += c * a.src_stride_of_dst_axis[i];
        }
        dst[t] = src[off];
    }
}

// dst[b][c][r] = src[b][r][c] for src [batch][R][Ccols]; 32x32 tiles through LDS with a
// +1 pad so the column read of the tile is bank-conflict free.
__global__ void __launch_bounds__(256) transpose_kernel(const float *__restrict__ src,
                                                          float *__restrict__ dst, int R, int Cc,
                                                          int tiles_c) {
    __shared__ float tile[32][33];
    const int b = blockIdx.y;
    const int tr = blockIdx.x / tiles_c;
    const int tc = blockIdx.x % tiles_c;
    const int tx = threadIdx.x & 31;
    const int ty = threadIdx.x >> 5;  // 0..7
    const float *s = src + (int64_t)b * R * Cc;
    float *d = dst + (int64_t)b * R * Cc;
#pragma unroll
    for (int j = 0; j < 32; j += 8) {
        const int r = tr * 32 + ty + j;
        const int c = tc * 32 + tx;
        if (r < R && c < Cc) tile[ty + j][tx] = s[(int64_t)r * Cc + c];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 32; j += 8) {
        const int c = tc * 32 + ty + j;
        const int r = tr * 32 + tx;
        if (r < R && c < Cc) d[(int64_t)c * R + r] = tile[tx][ty + j];
    }
}

// Sum over the middle axis of X[outer][axis][inner], in chunks of `rows` consecutive a:
//   out[c][o][i] = sum over a in [c*rows, min((c+1)*rows, axis)), ascending from +0.0f,
//                  of X[(o*axis + a)*inner + i].
// The reference kernels (cs/cl_kernels/reduce_sum_axis.cl:3-27, linear.cl:149-168) run one
// ascending chain per output over the whole axis: a single dependent chain per column,
// which at 12000 rows leaves the GPU waiting on one load at a time. With one chunk (axis <=
// rows) this is exactly the reference's order; otherwise the chunk sums are added in
// chunk order by reduce_slices_kernel (deterministic, and within the blocked-summation
// error bound (rows - 1 + chunks - 1) * 2^-24 * sum |x|). Each thread owns VW consecutive i
// (128-bit loads when VW = 4) and keeps CS_INFLIGHT rows of loads in flight. With
// `accumulate` (one chunk only) the sum is added to the output's value: out += sum.
constexpr int CS_INFLIGHT = 16;

template <int VW>
__global__ void __launch_bounds__(256) column_sum_kernel(const float *__restrict__ X,
                                                           float *__restrict__ out, int outer,
                                                           int axis, int inner, int rows,
                                                           int accumulate) {
    typedef float vec __attribute__((ext_vector_type(VW)));
    const int vecs = (inner + VW - 1) / VW;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)outer * vecs) return;
    // 32-bit division where it fits (a 64-bit one is a long software sequence)
    const int o = t <= INT32_MAX ? (int)((uint32_t)t / (uint32_t)vecs) : (int)(t / vecs);
    const int i0 = (int)(t - (int64_t)o * vecs) * VW;
    const int cnt = inner - i0 < VW ? inner - i0 : VW;
    const int c = blockIdx.y;
    const int a0 = c * rows;
    const int a1 = axis - a0 < rows ? axis : a0 + rows;
    const float *x = X + ((int64_t)o * axis + a0) * inner + i0;
    vec sum = {};
    if (cnt == VW) {
        for (int a = a0; a < a1; a += CS_INFLIGHT) {
            vec v[CS_INFLIGHT];
#pragma unroll
            for (int g = 0; g < CS_INFLIGHT; ++g)
                if (a + g < a1)
                    __builtin_memcpy(&v[g], x + (int64_t)(a - a0 + g) * inner, sizeof(vec));
#pragma unroll
            for (int g = 0; g < CS_INFLIGHT; ++g)
                if (a + g < a1) sum += v[g];
        }
    } else {
        for (int e = 0; e < cnt; ++e) {
            float s = 0.0f;
            for (int a = a0; a < a1; ++a) s += x[(int64_t)(a - a0) * inner + e];
            sum[e] = s;
        }
    }
    float *y = out + ((int64_t)c * outer + o) * inner + i0;
#pragma unroll
    for (int e = 0; e < VW; ++e)
        if (e < cnt) y[e] = accumulate ? y[e] + sum[e] : sum[e];
}

// Hp[t][h] = H[t - 1][h] when step t % seq_len > 0 of its sequence, else 0: the previous
// hidden state of the same sequence, the left operand of grad_U += H_prev^T * grad_gates
// (cs/cl_kernels/lstm.cl:582-590, tokens ordered [batch][seq_len]). VW consecutive h per
// thread (hidden % VW == 0).
template <int VW>
__global__ void __launch_bounds__(256) shift_rows_kernel(const float *__restrict__ H,
                                                           float *__restrict__ Hp,
                                                           int64_t total, int seq_len,
                                                           int hidden) {
    typedef float vec __attribute__((ext_vector_type(VW)));
    const int64_t step = (int64_t)gridDim.x * blockDim.x * VW;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VW; i < total;
         i += step) {
        // token index, by 32-bit division where it fits
        const int64_t t = i <= INT32_MAX ? (int64_t)((uint32_t)i / (uint32_t)hidden) : i / hidden;
        const int step_in_seq = t <= INT32_MAX ? (int)((uint32_t)t % (uint32_t)seq_len)
                                               : (int)(t % seq_len);
        vec v = {};
        if (step_in_seq != 0) __builtin_memcpy(&v, H + i - hidden, sizeof(vec));
        __builtin_memcpy(Hp + i, &v, sizeof(vec));
    }
}

// The streaming-read reference of the HBM-bound kernels (the GEMV of BASELINE config 5b):
// reads n4 float4 once, each work-group a contiguous range, every lane RS_U 16-byte
// non-temporal loads in flight, and writes one sum per work-group so the loads stay live.
// What it reaches is the read rate a kernel that only streams can get on the box.
constexpr int RS_U = 16;
__global__ void __launch_bounds__(256) stream_read_kernel(const float4 *__restrict__ src,
                                                          int64_t n4, int64_t per,
                                                          float *__restrict__ sums) {
    typedef float vec __attribute__((ext_vector_type(4)));
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = lo + per < n4 ? lo + per : n4;
    const vec *s = reinterpret_cast<const vec *>(src);
    vec acc = vec{0.f, 0.f, 0.f, 0.f};
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256 * RS_U) {
        vec v[RS_U];
#pragma unroll
        for (int u = 0; u < RS_U; ++u) {
            const int64_t j = i + (int64_t)u * 256;
            v[u] = j < hi ? __builtin_nontemporal_load(s + j) : vec{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < RS_U; ++u) acc += v[u];
    }
    __shared__ float part[256];
    part[threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) sums[blockIdx.x] = part[0];
}

}  // namespace

int launch_stream_read(hipStream_t stream, const float *src, int64_t n4, float *sums,
                       int blocks) {
    const int64_t per = (n4 + blocks - 1) / blocks;
    MIGEMM_LAUNCH(stream_read_kernel, dim3(blocks), dim3(256), 0, stream,
                  reinterpret_cast<const float4 *>(src), n4, per, sums);
    return launch_status("stream_read_kernel launch");
}

int launch_permute(hipStream_t stream, const float *src, float *dst, const int *src_dims,
                   const int *axes, int num_dims, int64_t total) {
    // Canonical form: size-1 axes dropped, and each run of destination axes that lie
    // consecutively and in order in the source merged into one axis (the outer one's source
    // stride is the inner one's stride times its size). [32,128,16,64] by (0,2,1,3) stays
    // 4-D; [B,R,C] by (0,2,1) is a batched transpose; an identity permutation is one axis.
    int64_t src_strides[MAXD];
    int64_t st = 1;
    for (int i = num_dims - 1; i >= 0; --i) {
        src_strides[i] = st;
        st *= src_dims[i];
    }
    int64_t cd[MAXD], cs[MAXD];
    int nd = 0;
    for (int i = 0; i < num_dims; ++i) {
        const int64_t d = src_dims[axes[i]];
        const int64_t str = src_strides[axes[i]];
        if (d == 1) continue;
        if (nd > 0 && cs[nd - 1] == str * d) {
            cd[nd - 1] *= d;
            cs[nd - 1] = str;
        } else {
            cd[nd] = d;
            cs[nd] = str;
            ++nd;
        }
    }
    if (nd == 0) {  // a single element
        cd[0] = 1;
        cs[0] = 1;
        nd = 1;
    }
    // Batched transpose of the last two axes with every leading axis in place: [R, C] ->
    // [C, R] is dst axes (C: stride 1, R: stride C), leading batch axis of stride R * C.
    const bool t2 = nd == 2 && cs[0] == 1 && cs[1] == cd[0];
    const bool t3 = nd == 3 && cs[1] == 1 && cs[2] == cd[1] && cs[0] == cd[1] * cd[2];
    if (t2 || t3) {
        const int64_t batch = t3 ? cd[0] : 1;
        const int64_t R = cd[nd - 1], Cc = cd[nd - 2];
        const int64_t tiles_r = (R + 31) / 32;
        const int64_t tiles_c = (Cc + 31) / 32;
        if (batch <= 65535 && R <= INT32_MAX && Cc <= INT32_MAX &&
            tiles_r * tiles_c <= INT32_MAX) {
            MIGEMM_LAUNCH(transpose_kernel, dim3((unsigned)(tiles_r * tiles_c),
                                                      (unsigned)batch),
                               dim3(256), 0, stream, src, dst, (int)R, (int)Cc, (int)tiles_c);
            record_plan(PlanRecord{"transpose", 32, 32, 1, 0, (int)R, (int)Cc, 0, (int)batch,
                                   false, false});
            return launch_status("transpose_kernel launch");
        }
    }
    // 16-byte elements when the innermost destination axis is the source's contiguous one
    // and holds whole groups of 4 (every other stride is then a multiple of 4 as well)
    const int vw = (cs[nd - 1] == 1 && cd[nd - 1] % 4 == 0 && ((uintptr_t)src & 15) == 0 &&
                    ((uintptr_t)dst & 15) == 0)
                       ? 4
                       : 1;
    PermuteArgs a;
    a.src = src;
    a.dst = dst;
    a.total = total / vw;
    a.ndim = nd;
    a.narrow = a.total <= INT32_MAX;
    for (int i = 0; i < MAXD; ++i) {
        a.dst_dims[i] = i < nd ? (i == nd - 1 ? cd[i] / vw : cd[i]) : 1;
        // in units of vw floats; with vw = 4 the innermost axis is contiguous (stride 1)
        a.src_stride_of_dst_axis[i] = i < nd ? cs[i] / (i == nd - 1 ? 1 : vw) : 0;
        a.div[i] = make_fastdiv(a.narrow ? (uint32_t)a.dst_dims[i] : 1u);
    }
    int64_t blocks = (a.total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (vw == 4)
        MIGEMM_LAUNCH(permute_gather_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream,
                           a);
    else
        MIGEMM_LAUNCH(permute_gather_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, stream,
                           a);
    record_plan(PlanRecord{"permute_gather", 0, 0, 1, 4 * vw, 0, 0, 0, nd, false, false});
    return launch_status("permute_gather_kernel launch");
}

int launch_column_sum(hipStream_t stream, const float *X, float *Y, int outer, int axis,
                      int inner, bool accumulate) {
    // Chunks of 256 rows: 12000 x 6565 (the Linear(500 -> 6565) bias gradient) is 47 chunks
    // of 7 work-groups, each thread with 16 rows of 128-bit loads in flight.
    int rows = 256;
    if ((axis + rows - 1) / rows > 65535) rows = (axis + 65534) / 65535;
    const int chunks = (axis + rows - 1) / rows;
    float *dst = Y;
    if (chunks > 1) {
        int st = MIGEMM_OK;
        dst = static_cast<float *>(
            workspace(stream, (size_t)chunks * outer * inner * sizeof(float), &st));
        if (dst == nullptr) return st;
    }
    const bool vec = inner % 4 == 0;
    const int64_t threads = (int64_t)outer * (vec ? inner / 4 : inner);
    const dim3 grid((unsigned)((threads + 255) / 256), (unsigned)chunks);
    if (vec)
        MIGEMM_LAUNCH(column_sum_kernel<4>, grid, dim3(256), 0, stream, X, dst, outer,
                           axis, inner, rows, (int)(accumulate && chunks == 1));
    else
        MIGEMM_LAUNCH(column_sum_kernel<1>, grid, dim3(256), 0, stream, X, dst, outer,
                           axis, inner, rows, (int)(accumulate && chunks == 1));
    const int rc = launch_status("column_sum_kernel launch");
    record_plan(PlanRecord{"column_sum", rows, vec ? 4 : 1, chunks, 0, outer, inner, axis, 1,
                           false, false});
    if (rc != MIGEMM_OK || chunks == 1) return rc;
    return launch_reduce_slices(stream, dst, chunks, outer, 1, inner, nullptr, Y, inner, inner,
                                accumulate);
}

int launch_shift_rows(hipStream_t stream, const float *H, float *Hp, int total_tokens,
                      int seq_len, int hidden) {
    const int64_t total = (int64_t)total_tokens * hidden;
    const bool vec = hidden % 4 == 0;
    int64_t blocks = ((vec ? total / 4 : total) + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (vec)
        MIGEMM_LAUNCH(shift_rows_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, H,
                           Hp, total, seq_len, hidden);
    else
        MIGEMM_LAUNCH(shift_rows_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, stream, H,
                           Hp, total, seq_len, hidden);
    return launch_status("shift_rows_kernel launch");
}

}  // namespace migemm
