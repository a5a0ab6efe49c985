/*
 * ref_runner.c -- runs the reference's own OpenCL kernels on the GPU. TEST INFRASTRUCTURE.
 *
 * The kernels are the reference sources (cl_kernels/matmul.cl, cl_kernels/permute.cl and
 * csharp/cstorchcl/cstorchcl/cl_kernels/bmm_permute_tiled.cl and linear.cl), compiled offline
 * by oracle/Makefile (target `ref`) with ROCm clang for gfx950 into oracle/_ref/ code objects and
 * loaded here with clCreateProgramWithBinary + clBuildProgram with no options, which is
 * what the reference hosts do with the source text (JITProgramCache.cs:33-34,
 * nncl_compiler.py:17: no build options, so FP_CONTRACT stays on and `acc += a*b` is an
 * fma). Launch geometry is the reference hosts':
 *   matmul_tiled       global (ceil(N/16)*16, ceil(M/16)*16)        local (16,16)
 *                      tests/test_matrix_ops.py:109-121
 *   bmm_tiled          global (ceil(N/16)*16, ceil(M/16)*16, batch) local (16,16,1)
 *                      csharp/.../compiler/NnClGlob.cs:472-478
 *   bmm_permute_tiled  global (ceil(N/64)*16, ceil(M/64)*16, batch) local (16,16,1)
 *                      NnClGlob.cs:1722-1748
 *   linear_forward_tiled  as bmm_permute_tiled                      NnClGlob.cs:1505-1543
 *   tensor_permute     global (total) local chosen by the driver    NnClGlob.cs:407-420
 *   lstm_gemm_xw       global (ceil(N/64)*16, ceil(M/64)*16) local (16,16)  NnClGlob.cs:891-899
 *   lstm_gemm_grad_x   global (ceil(F/64)*16, ceil(T/64)*16) local (16,16)  NnClGlob.cs:986-994
 *   lstm_gemm_grad_weights  global (ceil(4H/64)*16, ceil(max(F,H)/64)*16) local (16,16)
 *                      NnClGlob.cs:1017-1024
 *   lstm_recurrent_forward  global (wg, 1, batch) local (wg, 1, 1) with
 *                      wg = min(max work-group size, ceil(H/32)*32)  NnClGlob.cs:920-928
 *   lstm_hid_forward   global (batch) local chosen by the driver     NnClGlob.cs:1080-1097
 *
 * Usage: ref_runner <code_object> <kernel> <M> <K> <N> <batch> <sA> <sB> <sC> <transA>
 *                   <transB> <A.f32> <B.f32|-> <bias.f32|-> <out.f32> [reps]
 * (tensor_permute: M = num_dims, A = src, B = int32 file "dims then axes", K/N unused.
 *  lstm_gemm_xw: M = tokens, K = in_features, N = gates, A = X, B = W, bias.
 *  lstm_gemm_grad_x: M = tokens, K = gates, N = in_features, A = grad_gates, B = W.
 *  lstm_gemm_grad_weights: M = batch_size, K = seq_len, N = in_features, batch = hidden;
 *  A = X, B = H_out, bias = grad_gates; <out>.init holds the initial grad_W | grad_U |
 *  grad_bias, which are re-uploaded before every repetition (the kernel accumulates), and
 *  <out> receives the three concatenated.
 *  lstm_recurrent_forward: M = batch_size, K = seq_len, N = hidden; A = XW_in [B, S, 4H],
 *  B = U [H, 4H]; <out> receives H_out [B, S, H] followed by workspace [S, B, 5H].
 *  lstm_hid_forward: M = batch_size, K = seq_len, N = hidden, batch = in_features; A = X
 *  [B, S, F] then H_prev [B, H] then C_prev [B, H]; B = W [F, 4H] then U [H, 4H]; bias [4H];
 *  <out> receives H_out [B, S, H], workspace [S, B, 4H], final_H [B, H], final_C [B, H].)
 * Inputs are raw little-endian float32 files; the output file receives the kernel's output
 * buffer. One JSON line on stdout reports the median kernel time from OpenCL profiling
 * events. Exit status 3 means no OpenCL GPU device or the binary was refused (the caller
 * reports it as unavailable).
 */
#define CL_TARGET_OPENCL_VERSION 120
#include <CL/cl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void *read_file(const char *path, size_t *size) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *buf = malloc(n > 0 ? (size_t)n : 1);
    if (buf && n > 0 && fread(buf, 1, (size_t)n, f) != (size_t)n) {
        free(buf);
        buf = NULL;
    }
    fclose(f);
    *size = (size_t)n;
    return buf;
}

#define CHECK(x, what)                                                     \
    do {                                                                   \
        cl_int _e = (x);                                                   \
        if (_e != CL_SUCCESS) {                                            \
            fprintf(stderr, "ref_runner: %s failed (%d)\n", what, (int)_e); \
            return 2;                                                      \
        }                                                                  \
    } while (0)

static int cmp_double(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : x > y;
}

int main(int argc, char **argv) {
    if (argc < 16) {
        fprintf(stderr, "usage: see the header of ref_runner.c\n");
        return 1;
    }
    const char *co_path = argv[1], *kname = argv[2];
    const int M = atoi(argv[3]), K = atoi(argv[4]), N = atoi(argv[5]), batch = atoi(argv[6]);
    const int sA = atoi(argv[7]), sB = atoi(argv[8]), sC = atoi(argv[9]);
    const int transA = atoi(argv[10]), transB = atoi(argv[11]);
    const char *a_path = argv[12], *b_path = argv[13], *bias_path = argv[14];
    const char *out_path = argv[15];
    const int reps = argc > 16 ? atoi(argv[16]) : 3;

    cl_uint np = 0;
    if (clGetPlatformIDs(0, NULL, &np) != CL_SUCCESS || np == 0) {
        fprintf(stderr, "ref_runner: no OpenCL platform\n");
        return 3;
    }
    cl_platform_id plats[8];
    clGetPlatformIDs(np > 8 ? 8 : np, plats, NULL);
    cl_device_id dev = NULL;
    for (cl_uint i = 0; i < np && i < 8 && !dev; ++i) {
        cl_uint nd = 0;
        if (clGetDeviceIDs(plats[i], CL_DEVICE_TYPE_GPU, 1, &dev, &nd) != CL_SUCCESS || nd == 0)
            dev = NULL;
    }
    if (!dev) {
        fprintf(stderr, "ref_runner: no OpenCL GPU device\n");
        return 3;
    }
    char dname[256] = "";
    clGetDeviceInfo(dev, CL_DEVICE_NAME, sizeof(dname), dname, NULL);
    cl_int err;
    cl_context ctx = clCreateContext(NULL, 1, &dev, NULL, NULL, &err);
    CHECK(err, "clCreateContext");
    cl_command_queue q = clCreateCommandQueue(ctx, dev, CL_QUEUE_PROFILING_ENABLE, &err);
    CHECK(err, "clCreateCommandQueue");

    size_t co_size = 0;
    unsigned char *co = read_file(co_path, &co_size);
    if (!co) {
        fprintf(stderr, "ref_runner: cannot read %s\n", co_path);
        return 1;
    }
    const unsigned char *bins[1] = {co};
    cl_int bstat = CL_SUCCESS;
    cl_program prog = clCreateProgramWithBinary(ctx, 1, &dev, &co_size, bins, &bstat, &err);
    if (err != CL_SUCCESS || bstat != CL_SUCCESS) {
        fprintf(stderr, "ref_runner: binary refused (%d/%d)\n", (int)err, (int)bstat);
        return 3;
    }
    if (clBuildProgram(prog, 1, &dev, "", NULL, NULL) != CL_SUCCESS) {
        fprintf(stderr, "ref_runner: clBuildProgram failed\n");
        return 3;
    }
    cl_kernel kern = clCreateKernel(prog, kname, &err);
    CHECK(err, "clCreateKernel");

    size_t a_size = 0, b_size = 0, bias_size = 0;
    void *ha = read_file(a_path, &a_size);
    void *hb = strcmp(b_path, "-") ? read_file(b_path, &b_size) : NULL;
    void *hbias = strcmp(bias_path, "-") ? read_file(bias_path, &bias_size) : NULL;
    if (!ha) {
        fprintf(stderr, "ref_runner: cannot read inputs\n");
        return 1;
    }

    const int is_permute = strcmp(kname, "tensor_permute") == 0;
    const int is_gw = strcmp(kname, "lstm_gemm_grad_weights") == 0;
    const int is_rec = strcmp(kname, "lstm_recurrent_forward") == 0;
    const int is_hid = strcmp(kname, "lstm_hid_forward") == 0;
    /* lstm_hid_forward (M = batch, K = seq, N = hidden, batch = in_features): H_out,
     * workspace, final_H, final_C */
    const size_t hid_n[4] = {(size_t)M * K * N, (size_t)K * M * 4 * (size_t)N, (size_t)M * N,
                             (size_t)M * N};
    /* lstm_recurrent_forward: H_out [B, S, H] then workspace [S, B, 5H] */
    const size_t rec_n[2] = {(size_t)M * K * N, (size_t)K * M * 5 * (size_t)N};
    size_t out_elems;
    /* lstm_gemm_grad_weights: sizes of grad_W, grad_U, grad_bias */
    const size_t gw_n[3] = {(size_t)N * 4 * (size_t)batch, (size_t)batch * 4 * (size_t)batch,
                            4 * (size_t)batch};
    void *hinit = NULL;
    if (is_permute) {
        out_elems = a_size / sizeof(float);
    } else if (is_rec) {
        out_elems = rec_n[0] + rec_n[1];
    } else if (is_hid) {
        out_elems = hid_n[0] + hid_n[1] + hid_n[2] + hid_n[3];
        const size_t F = (size_t)batch, H = (size_t)N, Bn = (size_t)M, S = (size_t)K;
        if (a_size != (Bn * S * F + 2 * Bn * H) * sizeof(float) || !hb ||
            b_size != (F + H) * 4 * H * sizeof(float) || !hbias ||
            bias_size != 4 * H * sizeof(float)) {
            fprintf(stderr, "ref_runner: lstm_hid_forward input sizes do not match\n");
            return 1;
        }
    } else if (is_gw) {
        out_elems = gw_n[0] + gw_n[1] + gw_n[2];
        char init_path[4096];
        snprintf(init_path, sizeof(init_path), "%s.init", out_path);
        size_t init_size = 0;
        hinit = read_file(init_path, &init_size);
        if (!hinit || init_size != out_elems * sizeof(float)) {
            fprintf(stderr, "ref_runner: bad %s\n", init_path);
            return 1;
        }
    } else {
        out_elems = (size_t)(batch - 1) * (size_t)sC + (size_t)M * (size_t)N;
    }
    cl_mem da = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR, a_size, ha, &err);
    CHECK(err, "buffer A");
    cl_mem db = NULL, dbias = NULL, ddims = NULL, daxes = NULL, dsrcd = NULL;
    if (hb && !is_permute) {
        db = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR, b_size, hb, &err);
        CHECK(err, "buffer B");
    }
    if (hbias) {
        dbias = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR, bias_size, hbias,
                               &err);
        CHECK(err, "buffer bias");
    }
    cl_mem dc = clCreateBuffer(ctx, CL_MEM_READ_WRITE, out_elems * sizeof(float), NULL, &err);
    CHECK(err, "buffer C");

    cl_mem gw_bufs[3] = {NULL, NULL, NULL};
    cl_mem rec_ws = NULL;
    cl_mem hid_bufs[4] = {NULL, NULL, NULL, NULL}; /* H_out (= C), workspace, final_H, final_C */
    size_t gsz[3], lsz[3];
    cl_uint dims = 3;
    size_t *lptr = lsz;
    int t = 0;
    if (strcmp(kname, "matmul_tiled") == 0) {
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        dims = 2;
        gsz[0] = (size_t)((N + 15) / 16) * 16;
        gsz[1] = (size_t)((M + 15) / 16) * 16;
        lsz[0] = lsz[1] = 16;
    } else if (strcmp(kname, "bmm_tiled") == 0) {
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        clSetKernelArg(kern, t++, sizeof(int), &sA);
        clSetKernelArg(kern, t++, sizeof(int), &sB);
        clSetKernelArg(kern, t++, sizeof(int), &sC);
        gsz[0] = (size_t)((N + 15) / 16) * 16;
        gsz[1] = (size_t)((M + 15) / 16) * 16;
        gsz[2] = (size_t)batch;
        lsz[0] = lsz[1] = 16;
        lsz[2] = 1;
    } else if (strcmp(kname, "bmm_permute_tiled") == 0) {
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        clSetKernelArg(kern, t++, sizeof(int), &sA);
        clSetKernelArg(kern, t++, sizeof(int), &sB);
        clSetKernelArg(kern, t++, sizeof(int), &sC);
        clSetKernelArg(kern, t++, sizeof(int), &transA);
        clSetKernelArg(kern, t++, sizeof(int), &transB);
        gsz[0] = (size_t)((N + 63) / 64) * 16;
        gsz[1] = (size_t)((M + 63) / 64) * 16;
        gsz[2] = (size_t)batch;
        lsz[0] = lsz[1] = 16;
        lsz[2] = 1;
    } else if (strcmp(kname, "linear_forward_tiled") == 0) {
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dbias);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        clSetKernelArg(kern, t++, sizeof(int), &sA);
        clSetKernelArg(kern, t++, sizeof(int), &sC);
        gsz[0] = (size_t)((N + 63) / 64) * 16;
        gsz[1] = (size_t)((M + 63) / 64) * 16;
        gsz[2] = (size_t)batch;
        lsz[0] = lsz[1] = 16;
        lsz[2] = 1;
    } else if (strcmp(kname, "lstm_gemm_xw") == 0) {
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dbias);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        dims = 2;
        gsz[0] = (size_t)((N + 63) / 64) * 16;
        gsz[1] = (size_t)((M + 63) / 64) * 16;
        lsz[0] = lsz[1] = 16;
    } else if (strcmp(kname, "lstm_gemm_grad_x") == 0) {
        /* (all_grad_gates, W, grad_X, total_tokens, in_features, total_gates) */
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        dims = 2;
        gsz[0] = (size_t)((N + 63) / 64) * 16;
        gsz[1] = (size_t)((M + 63) / 64) * 16;
        lsz[0] = lsz[1] = 16;
    } else if (is_gw) {
        /* (X, H_out, all_grad_gates, grad_W, grad_U, grad_bias, batch, seq, in, hidden) */
        const int hidden = batch;
        /* grad_W lives in the output buffer C; grad_U and grad_bias get buffers of their own */
        cl_mem dgu = clCreateBuffer(ctx, CL_MEM_READ_WRITE, gw_n[1] * sizeof(float), NULL, &err);
        CHECK(err, "buffer grad_U");
        cl_mem dgb = clCreateBuffer(ctx, CL_MEM_READ_WRITE, gw_n[2] * sizeof(float), NULL, &err);
        CHECK(err, "buffer grad_bias");
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dbias);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dgu);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dgb);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        clSetKernelArg(kern, t++, sizeof(int), &hidden);
        gw_bufs[0] = dc;
        gw_bufs[1] = dgu;
        gw_bufs[2] = dgb;
        const int rows = N > hidden ? N : hidden;
        dims = 2;
        gsz[0] = (size_t)((4 * hidden + 63) / 64) * 16;
        gsz[1] = (size_t)((rows + 63) / 64) * 16;
        lsz[0] = lsz[1] = 16;
    } else if (is_rec) {
        /* (XW_in, U, H_out, workspace, batch_size, seq_len, hidden_size); H_out lives in the
         * output buffer C, the workspace gets a buffer of its own */
        rec_ws = clCreateBuffer(ctx, CL_MEM_READ_WRITE, rec_n[1] * sizeof(float), NULL, &err);
        CHECK(err, "buffer workspace");
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &db);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &rec_ws);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &N);
        size_t max_wg = 256;
        clGetDeviceInfo(dev, CL_DEVICE_MAX_WORK_GROUP_SIZE, sizeof(max_wg), &max_wg, NULL);
        size_t wg = (size_t)((N + 31) / 32) * 32;
        if (wg > max_wg) wg = max_wg;
        gsz[0] = wg;
        gsz[1] = 1;
        gsz[2] = (size_t)M;
        lsz[0] = wg;
        lsz[1] = lsz[2] = 1;
    } else if (is_hid) {
        /* (X, W, U, bias, H_prev, C_prev, H_out, workspace, final_H, final_C, batch, seq,
         * in, hidden); the inputs are slices of the A and B files */
        const int F = batch, H = N;
        const float *fa = (const float *)ha, *fb = (const float *)hb;
        const size_t nx = (size_t)M * K * F, nh = (size_t)M * H, nw = (size_t)F * 4 * H,
                     nu = (size_t)H * 4 * H;
        cl_mem in_bufs[5];
        const float *in_src[5] = {fa, fb, fb + nw, fa + nx, fa + nx + nh};
        const size_t in_n[5] = {nx, nw, nu, nh, nh};
        for (int i = 0; i < 5; ++i) {
            in_bufs[i] = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR,
                                        in_n[i] * sizeof(float), (void *)in_src[i], &err);
            CHECK(err, "lstm_hid_forward input");
        }
        hid_bufs[0] = dc;
        for (int i = 1; i < 4; ++i) {
            hid_bufs[i] = clCreateBuffer(ctx, CL_MEM_READ_WRITE, hid_n[i] * sizeof(float), NULL,
                                         &err);
            CHECK(err, "lstm_hid_forward output");
        }
        clSetKernelArg(kern, t++, sizeof(cl_mem), &in_bufs[0]); /* X */
        clSetKernelArg(kern, t++, sizeof(cl_mem), &in_bufs[1]); /* W */
        clSetKernelArg(kern, t++, sizeof(cl_mem), &in_bufs[2]); /* U */
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dbias);      /* bias */
        clSetKernelArg(kern, t++, sizeof(cl_mem), &in_bufs[3]); /* H_prev */
        clSetKernelArg(kern, t++, sizeof(cl_mem), &in_bufs[4]); /* C_prev */
        for (int i = 0; i < 4; ++i) clSetKernelArg(kern, t++, sizeof(cl_mem), &hid_bufs[i]);
        clSetKernelArg(kern, t++, sizeof(int), &M);
        clSetKernelArg(kern, t++, sizeof(int), &K);
        clSetKernelArg(kern, t++, sizeof(int), &F);
        clSetKernelArg(kern, t++, sizeof(int), &H);
        dims = 1;
        gsz[0] = (size_t)M;
        lptr = NULL;
    } else if (is_permute) {
        /* B file holds int32 dims[M] then axes[M]; M = num_dims */
        const int nd = M;
        const int *meta = (const int *)hb;
        if (!meta || b_size < 2 * (size_t)nd * sizeof(int)) {
            fprintf(stderr, "ref_runner: bad permute metadata\n");
            return 1;
        }
        int dst_dims[10];
        for (int i = 0; i < nd; ++i) dst_dims[i] = meta[meta[nd + i]];
        dsrcd = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR, nd * sizeof(int),
                               (void *)meta, &err);
        CHECK(err, "src dims");
        ddims = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR, nd * sizeof(int),
                               dst_dims, &err);
        CHECK(err, "dst dims");
        daxes = clCreateBuffer(ctx, CL_MEM_READ_ONLY | CL_MEM_COPY_HOST_PTR, nd * sizeof(int),
                               (void *)(meta + nd), &err);
        CHECK(err, "axes");
        const int total = (int)out_elems;
        clSetKernelArg(kern, t++, sizeof(cl_mem), &da);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dc);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &dsrcd);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &ddims);
        clSetKernelArg(kern, t++, sizeof(cl_mem), &daxes);
        clSetKernelArg(kern, t++, sizeof(int), &nd);
        clSetKernelArg(kern, t++, sizeof(int), &total);
        dims = 1;
        gsz[0] = out_elems;
        lptr = NULL;
    } else {
        fprintf(stderr, "ref_runner: unknown kernel %s\n", kname);
        return 1;
    }

    double times[64];
    int nrep = reps < 1 ? 1 : (reps > 64 ? 64 : reps);
    for (int r = 0; r < nrep; ++r) {
        if (is_gw) {
            /* the kernel accumulates: every repetition starts from the initial values */
            const float *init = (const float *)hinit;
            size_t off = 0;
            for (int i = 0; i < 3; ++i) {
                CHECK(clEnqueueWriteBuffer(q, gw_bufs[i], CL_TRUE, 0, gw_n[i] * sizeof(float),
                                           init + off, 0, NULL, NULL),
                      "upload init");
                off += gw_n[i];
            }
        }
        cl_event ev;
        CHECK(clEnqueueNDRangeKernel(q, kern, dims, NULL, gsz, lptr, 0, NULL, &ev), "enqueue");
        CHECK(clFinish(q), "clFinish");
        cl_ulong t0 = 0, t1 = 0;
        clGetEventProfilingInfo(ev, CL_PROFILING_COMMAND_START, sizeof(t0), &t0, NULL);
        clGetEventProfilingInfo(ev, CL_PROFILING_COMMAND_END, sizeof(t1), &t1, NULL);
        times[r] = (double)(t1 - t0) * 1e-3;
        clReleaseEvent(ev);
    }
    qsort(times, (size_t)nrep, sizeof(double), cmp_double);
    float *hc = malloc(out_elems * sizeof(float));
    if (is_gw) {
        size_t off = 0;
        for (int i = 0; i < 3; ++i) {
            CHECK(clEnqueueReadBuffer(q, gw_bufs[i], CL_TRUE, 0, gw_n[i] * sizeof(float),
                                      hc + off, 0, NULL, NULL),
                  "read grads");
            off += gw_n[i];
        }
    } else if (is_hid) {
        size_t off = 0;
        for (int i = 0; i < 4; ++i) {
            CHECK(clEnqueueReadBuffer(q, hid_bufs[i], CL_TRUE, 0, hid_n[i] * sizeof(float),
                                      hc + off, 0, NULL, NULL),
                  "read lstm_hid_forward outputs");
            off += hid_n[i];
        }
    } else if (is_rec) {
        CHECK(clEnqueueReadBuffer(q, dc, CL_TRUE, 0, rec_n[0] * sizeof(float), hc, 0, NULL,
                                  NULL),
              "read H_out");
        CHECK(clEnqueueReadBuffer(q, rec_ws, CL_TRUE, 0, rec_n[1] * sizeof(float),
                                  hc + rec_n[0], 0, NULL, NULL),
              "read workspace");
    } else {
        CHECK(clEnqueueReadBuffer(q, dc, CL_TRUE, 0, out_elems * sizeof(float), hc, 0, NULL,
                                  NULL),
              "read C");
    }
    FILE *f = fopen(out_path, "wb");
    if (!f || fwrite(hc, sizeof(float), out_elems, f) != out_elems) {
        fprintf(stderr, "ref_runner: cannot write %s\n", out_path);
        return 1;
    }
    fclose(f);
    printf("{\"kernel\": \"%s\", \"device\": \"%s\", \"median_us\": %.3f, \"reps\": %d}\n", kname,
           dname, times[nrep / 2], nrep);
    return 0;
}
