/* g4gpu.h -- the optional GPU backend for model.c's matmul_b that
 * INTEGRATION.md shows a maintainer adding to g4run (g4gpu.c). */
#ifndef G4GPU_H
#define G4GPU_H
#include <stdint.h>

#include "g4hip.h"
#include "g4run_abi.h"

typedef struct {            /* one per uploaded g4_tensor */
    g4h_tensor *t;
} g4gpu_weight;

int  g4gpu_init(int device);
int  g4gpu_upload(const g4_tensor *w, g4gpu_weight *out);
void g4gpu_release(g4gpu_weight *w);
/* drop-in for matmul_b(c, wtype, W, x, NULL, 0, Y, ncols, nrows, nb) with host
 * x [nb][ncols] and Y [nb][nrows] (model.c:257-270); 0 on success */
int  g4gpu_matmul(const g4gpu_weight *W, const float *x, float *Y, int64_t ncols, int64_t nrows, int nb);
#endif
