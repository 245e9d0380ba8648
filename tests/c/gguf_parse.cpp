// gguf_parse.cpp -- opens each GGUF file named on the command line with the
// library's parser (g4run_amd/csrc/gguf.cpp + types.cpp, built together with
// this file under AddressSanitizer and UBSan) and prints one line per file:
// "1" if it parsed, "0" if the parser refused it, "bounds <name>" for a
// parsed tensor whose data is not inside the file's mapping (the parser's
// bounds check, gguf.c:395-404, must make that impossible).
#include <cstdint>
#include <cstdio>

#include "../../include/g4run_abi.h"

int main(int argc, char **argv) {
    for (int i = 1; i < argc; i++) {
        g4_model_file mf;
        if (g4_gguf_open(&mf, argv[i], false) != 0) {
            printf("0\n");
            continue;
        }
        const uint8_t *lo = (const uint8_t *)mf.map_base, *hi = lo + mf.map_size;
        bool ok = true;
        unsigned sum = 0;
        for (uint64_t k = 0; k < mf.n_tensors; k++) {
            const g4_tensor &t = mf.tensors[k];
            uint64_t rows = 1;
            for (int d = 1; d < t.ndim && d < 4; d++) rows *= (uint64_t)t.ne[d];
            const uint64_t bytes = rows * g4_row_size(t.type, t.ne[0]);
            const uint8_t *p = (const uint8_t *)t.data;
            if (p < lo || p > hi || bytes > (uint64_t)(hi - p)) {
                printf("bounds %s\n", t.name);
                ok = false;
                break;
            }
            if (bytes) sum += p[0] + p[bytes - 1];               // the first and last byte of the data
        }
        g4_gguf_close(&mf);
        if (ok) printf("1\n");
        fflush(stdout);
        (void)sum;
    }
    return 0;
}
