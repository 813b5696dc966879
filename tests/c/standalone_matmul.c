/* A C99 caller of the hip backend through the public scrapgpu_ C API only (include/scrapgpu/),
 * shaped like the reference's examples/standalone_matmul.c:115-195: register the backend, take
 * device 0, upload Q4_0 weights as R32, upload x, run MUL_MAT, download y.
 *
 *   standalone_matmul K M N w.bin x.bin y_out.bin
 *
 * w.bin holds the natural Q4_0 blocks of the M x K weights, x.bin N x K floats; y_out.bin receives
 * N x M floats. Exit status: 0 done, 2 no gfx950 device, 1 any failure (message on stderr). The
 * test that runs it computes the expected y with the CPU oracle (there is no CPU reference in the
 * library itself). */
#include "scrapgpu/api.h"
#include "scrapgpu/hip.h"
#include "scrapgpu/stream.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void die(const char * what, scrapgpu_status st) {
    fprintf(stderr, "%s: %s (%s)\n", what, scrapgpu_status_string(st), scrapgpu_last_error());
    exit(1);
}

static void * slurp(const char * path, size_t want) {
    FILE * f = fopen(path, "rb");
    if (f == NULL) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(1);
    }
    void * p = malloc(want ? want : 1);
    if (p == NULL || fread(p, 1, want, f) != want) {
        fprintf(stderr, "%s: expected %zu bytes\n", path, want);
        exit(1);
    }
    fclose(f);
    return p;
}

static scrapgpu_tensor_desc desc2d(scrapgpu_dtype dt, scrapgpu_buffer_t * b, int64_t ne0, int64_t ne1, scrapgpu_layout layout) {
    scrapgpu_tensor_desc t;
    memset(&t, 0, sizeof(t));
    t.struct_size = sizeof(t);
    t.dtype = dt;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = 1;
    t.ne[3] = 1;
    t.nb[0] = scrapgpu_dtype_type_size(dt);
    t.nb[1] = scrapgpu_tensor_row_size(dt, ne0);
    t.nb[2] = t.nb[1] * (uint64_t) ne1;
    t.nb[3] = t.nb[2];
    t.buffer = b;
    t.offset = 0;
    t.layout = layout;
    return t;
}

int main(int argc, char ** argv) {
    if (argc != 7) {
        fprintf(stderr, "usage: %s K M N w.bin x.bin y_out.bin\n", argv[0]);
        return 1;
    }
    const int64_t K = atoll(argv[1]), M = atoll(argv[2]), N = atoll(argv[3]);
    if (K <= 0 || K % 32 != 0 || M <= 0 || N <= 0) {
        fprintf(stderr, "K must be a positive multiple of 32, M and N positive\n");
        return 1;
    }
    scrapgpu_status st = scrapgpu_hip_register();
    if (st != SCRAPGPU_STATUS_OK) die("scrapgpu_hip_register", st);
    if (scrapgpu_get_device_count() == 0) {
        fprintf(stderr, "no gfx950 device\n");
        return 2;
    }
    scrapgpu_device_t * dev = NULL;
    if ((st = scrapgpu_get_device(0, &dev)) != SCRAPGPU_STATUS_OK) die("scrapgpu_get_device", st);
    scrapgpu_device_info info;
    scrapgpu_device_info_init(&info, sizeof(info));
    if ((st = scrapgpu_device_get_info(dev, &info)) != SCRAPGPU_STATUS_OK) die("scrapgpu_device_get_info", st);
    scrapgpu_stream_t * stream = NULL;
    if ((st = scrapgpu_stream_create(dev, &stream)) != SCRAPGPU_STATUS_OK) die("scrapgpu_stream_create", st);

    const size_t w_bytes = scrapgpu_tensor_row_size(SCRAPGPU_DTYPE_Q4_0, K) * (size_t) M;
    void * wq = slurp(argv[4], w_bytes);
    float * x = (float *) slurp(argv[5], (size_t) K * N * sizeof(float));
    float * y = (float *) malloc((size_t) M * N * sizeof(float));

    scrapgpu_buffer_t *bw = NULL, *bx = NULL, *by = NULL;
    if ((st = scrapgpu_buffer_alloc(dev, w_bytes, &bw)) != SCRAPGPU_STATUS_OK) die("buffer_alloc w", st);
    if ((st = scrapgpu_buffer_alloc(dev, (size_t) K * N * 4, &bx)) != SCRAPGPU_STATUS_OK) die("buffer_alloc x", st);
    if ((st = scrapgpu_buffer_alloc(dev, (size_t) M * N * 4, &by)) != SCRAPGPU_STATUS_OK) die("buffer_alloc y", st);

    /* the upload repacks the natural blocks into R32 on the device */
    scrapgpu_tensor_desc w = desc2d(SCRAPGPU_DTYPE_Q4_0, bw, K, M, SCRAPGPU_LAYOUT_R32);
    scrapgpu_tensor_desc xt = desc2d(SCRAPGPU_DTYPE_F32, bx, K, N, SCRAPGPU_LAYOUT_NATURAL);
    scrapgpu_tensor_desc yt = desc2d(SCRAPGPU_DTYPE_F32, by, M, N, SCRAPGPU_LAYOUT_NATURAL);
    if ((st = scrapgpu_tensor_upload(stream, &w, wq, w_bytes)) != SCRAPGPU_STATUS_OK) die("upload w", st);
    if ((st = scrapgpu_tensor_upload(stream, &xt, x, (size_t) K * N * 4)) != SCRAPGPU_STATUS_OK) die("upload x", st);

    const scrapgpu_tensor_desc ins[2] = {w, xt};
    scrapgpu_mul_mat_params mm;
    memset(&mm, 0, sizeof(mm));
    mm.struct_size = sizeof(mm);
    scrapgpu_op_desc op;
    memset(&op, 0, sizeof(op));
    op.struct_size = sizeof(op);
    op.op = SCRAPGPU_OP_MUL_MAT;
    op.inputs = ins;
    op.input_count = 2;
    op.outputs = &yt;
    op.output_count = 1;
    op.params = &mm;
    op.params_size = sizeof(mm);

    const char * reason = NULL;
    if ((st = scrapgpu_op_supported(dev, &op, &reason)) != SCRAPGPU_STATUS_OK) {
        fprintf(stderr, "MUL_MAT is not supported: %s\n", reason ? reason : "?");
        return 1;
    }
    if ((st = scrapgpu_op_execute(stream, &op)) != SCRAPGPU_STATUS_OK) die("op_execute", st);
    if ((st = scrapgpu_stream_sync(stream)) != SCRAPGPU_STATUS_OK) die("stream_sync", st);
    if ((st = scrapgpu_tensor_download(stream, &yt, y, (size_t) M * N * 4)) != SCRAPGPU_STATUS_OK) die("download y", st);

    FILE * f = fopen(argv[6], "wb");
    if (f == NULL || fwrite(y, sizeof(float), (size_t) M * N, f) != (size_t) M * N) {
        fprintf(stderr, "cannot write %s\n", argv[6]);
        return 1;
    }
    fclose(f);
    printf("MUL_MAT Q4_0(R32) [%lld x %lld] x [%lld x %lld] on %s (%s)\n", (long long) K, (long long) M, (long long) K, (long long) N,
           info.name ? info.name : "?", info.backend_name ? info.backend_name : "?");

    scrapgpu_buffer_free(bw);
    scrapgpu_buffer_free(bx);
    scrapgpu_buffer_free(by);
    scrapgpu_stream_free(stream);
    free(wq);
    free(x);
    free(y);
    return 0;
}
