/* g4gpu.c -- optional GPU backend for matmul_b, linked with -lg4hip (the
 * listing of INTEGRATION.md section 2, compiled and run by the GPU tests). */
#include "g4gpu.h"

#include <stdio.h>

static void *g4gpu_stream;                 /* NULL = the null stream */
static float *g4gpu_x, *g4gpu_y;           /* device staging for x / Y */
static size_t g4gpu_cap_x, g4gpu_cap_y;

int g4gpu_init(int device) {
    int rc = g4h_init(device);
    if (rc) fprintf(stderr, "g4gpu: %s\n", g4h_last_error());
    return rc;
}

/* once per weight matrix, after gguf load: copy to HBM and repack */
int g4gpu_upload(const g4_tensor *w, g4gpu_weight *out) {
    int64_t ncols = w->ne[0], nrows = w->ne[1];
    int rc = g4h_tensor_create(w->type, ncols, nrows, &out->t);
    if (!rc) rc = g4h_tensor_load(out->t, w->data, /*src_is_device=*/0, g4gpu_stream);
    if (!rc) rc = g4h_stream_synchronize(g4gpu_stream);
    return rc;
}

void g4gpu_release(g4gpu_weight *w) {
    g4h_tensor_free(w->t);
    w->t = NULL;
}

static int grow(void **p, size_t *cap, size_t need) {
    if (*cap >= need) return G4H_OK;
    g4h_free(*p);
    *cap = 0;
    int rc = g4h_malloc(p, need);
    if (!rc) *cap = need;
    return rc;
}

int g4gpu_matmul(const g4gpu_weight *W, const float *x, float *Y, int64_t ncols, int64_t nrows, int nb) {
    int rc = grow((void **)&g4gpu_x, &g4gpu_cap_x, (size_t)nb * ncols * 4);
    if (!rc) rc = grow((void **)&g4gpu_y, &g4gpu_cap_y, (size_t)nb * nrows * 4);
    if (!rc) rc = g4h_memcpy_h2d(g4gpu_x, x, (size_t)nb * ncols * 4, g4gpu_stream);
    if (!rc) rc = g4h_matmul(W->t, g4gpu_x, NULL, 0, g4gpu_y, nb, g4gpu_stream);
    if (!rc) rc = g4h_memcpy_d2h(Y, g4gpu_y, (size_t)nb * nrows * 4, g4gpu_stream);  /* synchronizes */
    if (rc) fprintf(stderr, "g4gpu_matmul: %s (%s)\n", g4h_last_error(), g4h_status_str(rc));
    return rc;
}
