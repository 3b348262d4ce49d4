/*
 * abi_caller.c -- a C program that uses libqmoe.so only through
 * include/qmoe.h, the way the reference C port would call it in place of its
 * MoE layer (c/src/model.c:1712): create a context sized like moe_forward's
 * scratch (model.c:1593-1596), upload one layer from host arrays in the
 * checkpoint layout (what mw_load / experts_load hold, model.c:213-272,
 * 539-674), then run the layer
 *   (a) with moe_forward's host fp32 contract (qmoe_moe_forward_host), and
 *   (b) on device buffers (qmoe_layer_forward + qmoe_last_routing),
 * and compare both with the expected output and routing of the fixture.
 *
 *   abi_caller --version          prints the library version (no GPU call)
 *   abi_caller FIXTURE            runs the layer; exit status 0 when every
 *                                 check passes
 *
 * FIXTURE (little endian): the 8 bytes "QMOEFIX1", int32 H, E, k, I, n,
 * then int64 byte count + bytes for each of: router_w, gate_q, gate_s,
 * gate_b, up_q, up_s, up_b, down_q, down_s, down_b, sh_gate_q, sh_gate_s,
 * sh_gate_b, sh_up_q, sh_up_s, sh_up_b, sh_down_q, sh_down_s, sh_down_b,
 * sh_gate_w (checkpoint dtypes: u32 codes, bf16 bits), x [n,H] f32,
 * expected out [n,H] f32, expected top-k ids [n,k] int32.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "qmoe.h"

#define N_BLOBS 23

static void *read_blob(FILE *f, int64_t *bytes) {
    if (fread(bytes, 8, 1, f) != 1 || *bytes < 0 || *bytes > ((int64_t)1 << 32)) return NULL;
    void *p = malloc(*bytes ? (size_t)*bytes : 1);
    if (p && *bytes && fread(p, 1, (size_t)*bytes, f) != (size_t)*bytes) {
        free(p);
        return NULL;
    }
    return p;
}

static int compare(const char *what, const float *got, const float *ref, size_t count) {
    double num = 0.0, den = 0.0, mx = 0.0;
    for (size_t i = 0; i < count; i++) {
        const double d = (double)got[i] - (double)ref[i];
        num += d * d;
        den += (double)ref[i] * ref[i];
        if (fabs(d) > mx || d != d) mx = d != d ? INFINITY : fabs(d);
    }
    const double rel = sqrt(num / (den > 0 ? den : 1e-300));
    const int ok = mx < 2e-2 && rel < 1e-3;
    printf("%s: max-abs %.3e rel-L2 %.3e %s\n", what, mx, rel, ok ? "ok" : "FAIL");
    return ok ? 0 : 1;
}

int main(int argc, char **argv) {
    if (argc == 2 && !strcmp(argv[1], "--version")) {
        printf("%s\n", qmoe_version());
        return 0;
    }
    if (argc != 2) {
        fprintf(stderr, "usage: %s FIXTURE | --version\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "rb");
    if (!f) {
        perror(argv[1]);
        return 2;
    }
    char magic[8];
    int32_t dims[5];
    if (fread(magic, 1, 8, f) != 8 || memcmp(magic, "QMOEFIX1", 8) || fread(dims, 4, 5, f) != 5) {
        fprintf(stderr, "bad fixture header\n");
        return 2;
    }
    const int H = dims[0], E = dims[1], k = dims[2], I = dims[3], n = dims[4];
    void *blob[N_BLOBS];
    int64_t nb[N_BLOBS];
    for (int i = 0; i < N_BLOBS; i++) {
        blob[i] = read_blob(f, &nb[i]);
        if (!blob[i]) {
            fprintf(stderr, "fixture truncated at tensor %d\n", i);
            return 2;
        }
    }
    fclose(f);
    const float *x = (const float *)blob[20], *want = (const float *)blob[21];
    const int32_t *want_idx = (const int32_t *)blob[22];

    qmoe_err err;
    qmoe_ctx *ctx = NULL;
    const qmoe_config cfg = {H, E, k, I, 64, 1, n, 1e-6f};
    if (qmoe_create(&ctx, &cfg, &err)) {
        fprintf(stderr, "qmoe_create: %s\n", err.msg);
        return 1;
    }
    /* the layer as the C port holds it after loading (bf16 scales and
     * biases kept as stored; the port widens them to f32 at load) */
    qmoe_layer_weights w;
    memset(&w, 0, sizeof(w));
    w.router_w = blob[0];
    w.gate_q = blob[1];
    w.gate_s = blob[2];
    w.gate_b = blob[3];
    w.up_q = blob[4];
    w.up_s = blob[5];
    w.up_b = blob[6];
    w.down_q = blob[7];
    w.down_s = blob[8];
    w.down_b = blob[9];
    w.sh_gate_q = blob[10];
    w.sh_gate_s = blob[11];
    w.sh_gate_b = blob[12];
    w.sh_up_q = blob[13];
    w.sh_up_s = blob[14];
    w.sh_up_b = blob[15];
    w.sh_down_q = blob[16];
    w.sh_down_s = blob[17];
    w.sh_down_b = blob[18];
    w.sh_gate_w = blob[19];
    int fails = 0;
    if (qmoe_upload_layer(ctx, 0, &w, &err)) {
        fprintf(stderr, "qmoe_upload_layer: %s\n", err.msg);
        return 1;
    }

    /* (a) the host shim with moe_forward's data contract */
    float *out = (float *)malloc((size_t)n * H * sizeof(float));
    if (qmoe_moe_forward_host(ctx, 0, x, n, out, &err)) {
        fprintf(stderr, "qmoe_moe_forward_host: %s\n", err.msg);
        return 1;
    }
    fails += compare("moe_forward_host", out, want, (size_t)n * H);

    /* (b) device buffers on a caller stream */
    hipStream_t st;
    float *dx = NULL, *dout = NULL;
    int32_t *didx = NULL;
    if (hipStreamCreate(&st) || hipMalloc((void **)&dx, (size_t)n * H * 4) ||
        hipMalloc((void **)&dout, (size_t)n * H * 4) || hipMalloc((void **)&didx, (size_t)n * k * 4) ||
        hipMemcpy(dx, x, (size_t)n * H * 4, hipMemcpyHostToDevice)) {
        fprintf(stderr, "HIP set-up failed\n");
        return 1;
    }
    if (qmoe_layer_forward(ctx, 0, dx, QMOE_F32, n, dout, 0, st, &err) ||
        qmoe_last_routing(ctx, n, didx, NULL, NULL, NULL, NULL, NULL, st, &err)) {
        fprintf(stderr, "layer call: %s\n", err.msg);
        return 1;
    }
    int32_t *idx = (int32_t *)malloc((size_t)n * k * 4);
    float *out2 = (float *)malloc((size_t)n * H * 4);
    if (hipStreamSynchronize(st) || hipMemcpy(out2, dout, (size_t)n * H * 4, hipMemcpyDeviceToHost) ||
        hipMemcpy(idx, didx, (size_t)n * k * 4, hipMemcpyDeviceToHost)) {
        fprintf(stderr, "HIP copy-back failed\n");
        return 1;
    }
    fails += compare("layer_forward", out2, want, (size_t)n * H);
    const int same_ids = !memcmp(idx, want_idx, (size_t)n * k * 4);
    printf("top-k ids: %s\n", same_ids ? "bit-exact" : "FAIL");
    fails += !same_ids;
    const int same_bits = !memcmp(out, out2, (size_t)n * H * 4);
    printf("host shim == device call: %s\n", same_bits ? "bit-identical" : "FAIL");
    fails += !same_bits;

    /* the error convention: -1 and a message, nothing aborts */
    if (qmoe_moe_forward_host(ctx, 0, x, n + 1, out, &err) != -1 || !err.msg[0]) {
        printf("error path: FAIL\n");
        fails++;
    } else {
        printf("error path: ok (%s)\n", err.msg);
    }

    hipFree(dx);
    hipFree(dout);
    hipFree(didx);
    hipStreamDestroy(st);
    qmoe_destroy(ctx);
    for (int i = 0; i < N_BLOBS; i++) free(blob[i]);
    free(out);
    free(out2);
    free(idx);
    printf("%s\n", fails ? "FAILED" : "PASSED");
    return fails ? 1 : 0;
}
