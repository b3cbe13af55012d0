/* A C consumer of include/flashcqt.h: compiles as C99 against the header,
 * links libflashcqt.so and exercises the calls that need no GPU (version,
 * status strings, argument checks made before any HIP call), then loads a
 * table image file (argv[1], written by flash_cqt/tables.py save_image),
 * checks it and sizes every buffer for batch 64 from the library alone.
 * Exit 0 on success; prints the first failed check otherwise. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "flashcqt.h"

#define CHECK(cond)                                                   \
    do {                                                              \
        if (!(cond)) {                                                \
            fprintf(stderr, "check failed: %s (line %d)\n", #cond, __LINE__); \
            return 1;                                                 \
        }                                                             \
    } while (0)

int main(int argc, char** argv) {
    static float buf[64] __attribute__((aligned(16)));
    fcqt_tables tab;
    memset(&tab, 0, sizeof(tab));
    tab.tw_pass = buf;
    tab.tw_half = buf;
    tab.tw_stage = buf;
    tab.tasks = (const int32_t*)buf;
    tab.ntasks = 1;
    tab.ncoef = 1;
    tab.coef_span = 1;
    hipStream_t s = 0;

    CHECK(fcqt_abi_version() == FCQT_ABI_VERSION);
    CHECK(strcmp(fcqt_status_string(FCQT_OK), "ok") == 0);
    CHECK(strstr(fcqt_status_string(FCQT_EARG), "argument") != NULL);
    /* null buffers, batch 0, bad layout, misalignment: rejected before any launch */
    CHECK(fcqt_packed_fft_fwd(NULL, buf, buf, buf, 1, s) == FCQT_EARG);
    CHECK(fcqt_packed_fft_fwd(&tab, NULL, buf, buf, 1, s) == FCQT_EARG);
    CHECK(fcqt_packed_fft_fwd(&tab, buf, buf, buf, 0, s) == FCQT_EARG);
    CHECK(fcqt_packed_fft_fwd(&tab, buf + 1, buf, buf, 1, s) == FCQT_EALIGN);
    CHECK(fcqt_route_bands(&tab, (const int32_t*)buf, buf, buf, buf, 7, 1, s) == FCQT_EARG);
    CHECK(fcqt_scatter_bands(&tab, (const int32_t*)buf, buf, buf, FCQT_PLANAR, NULL, 1, s) == FCQT_EARG);
    CHECK(fcqt_packed_fft_inv(&tab, NULL, buf, buf, buf, 1, s) == FCQT_EARG);
    /* a task table reaching past the coefficient row is refused */
    tab.coef_span = 2;
    CHECK(fcqt_route_bands(&tab, (const int32_t*)buf, buf, buf, buf, FCQT_PLANAR, 1, s) == FCQT_EARG);
    CHECK(fcqt_scatter_bands(&tab, (const int32_t*)buf, buf, buf, FCQT_PLANAR, buf, 1, s) == FCQT_EARG);
    CHECK(fcqt_analysis(&tab, (const int32_t*)buf, buf, buf, buf, FCQT_PLANAR, buf, buf, 1, s) == FCQT_EARG);
    tab.coef_span = 1;
    CHECK(fcqt_fill_zero(NULL, 4, s) == FCQT_EARG);
    CHECK(fcqt_fill_zero(buf, 0, s) == FCQT_OK);
    CHECK(fcqt_stream_overlap(buf, NULL, buf, 1, 1, s) == FCQT_EARG);
    if (argc > 1) {
        FILE* fp = fopen(argv[1], "rb");
        CHECK(fp != NULL);
        fseek(fp, 0, SEEK_END);
        long len = ftell(fp);
        fseek(fp, 0, SEEK_SET);
        unsigned char* img = (unsigned char*)malloc((size_t)len);
        CHECK(img != NULL && fread(img, 1, (size_t)len, fp) == (size_t)len);
        fclose(fp);
        fcqt_image_info info;
        CHECK(fcqt_image_check(img, len, &info) == FCQT_OK);
        CHECK(info.device_bytes == len && info.ncoef == info.coef_span && info.ntasks > 0);
        img[0] = 'X';
        CHECK(fcqt_image_check(img, len, NULL) == FCQT_EARG);
        free(img);
        fcqt_tables t2;
        memset(&t2, 0, sizeof(t2));
        t2.ncoef = info.ncoef;
        fcqt_sizes sz;
        CHECK(fcqt_workspace_sizes(&t2, 64, &sz) == FCQT_OK);
        printf("image ok: %lld device bytes, ncoef %lld, %d tasks\n", (long long)info.device_bytes,
               (long long)info.ncoef, (int)info.ntasks);
        printf("batch 64 bytes: signal %lld spectrum %lld work %lld scatter %lld coef_plane %lld tail %lld sync %lld\n",
               (long long)sz.signal, (long long)sz.spectrum, (long long)sz.work, (long long)sz.scatter,
               (long long)sz.coef_plane, (long long)sz.tail, (long long)sz.sync);
    }
    printf("c abi check ok (ABI %d)\n", fcqt_abi_version());
    return 0;
}
