/* End-to-end C consumer of include/flashcqt.h: everything a C or C++
 * program needs to run the engine without Python.
 *   roundtrip <table image> <batch> <input: batch x 65536 float32, raw>
 *             <output: coefficients, raw float32 planes KR then KI>
 * Loads and checks the table image (written once by flash_cqt/tables.py
 * save_image), uploads it, sizes every buffer with fcqt_workspace_sizes,
 * allocates them with hipMalloc, runs the analysis and the synthesis on the
 * default stream, prints the round-trip SNR of every row and writes the
 * coefficients out. Then runs the same round trip through the single-launch
 * entry points (one launch per direction, a zero-filled stage-counter
 * buffer) and checks that they give the same bits and leave the counters and
 * the error word at zero. Exit 0 on success; prints the first failed call
 * otherwise. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "flashcqt.h"

#define HIPCHECK(x)                                                                     \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));              \
            return 1;                                                                   \
        }                                                                               \
    } while (0)
#define FCQT(x)                                                                         \
    do {                                                                                \
        int r_ = (x);                                                                   \
        if (r_) {                                                                       \
            fprintf(stderr, "%s failed: %s (%s)\n", #x, fcqt_status_string(r_), fcqt_last_hip_error()); \
            return 1;                                                                   \
        }                                                                               \
    } while (0)

static void* read_file(const char* path, long* len) {
    FILE* fp = fopen(path, "rb");
    if (!fp) return NULL;
    void* buf = NULL;
    if (fseek(fp, 0, SEEK_END) == 0) {
        *len = ftell(fp);
        if (*len > 0 && fseek(fp, 0, SEEK_SET) == 0) {
            buf = malloc((size_t)*len);
            if (buf && fread(buf, 1, (size_t)*len, fp) != (size_t)*len) {
                free(buf);
                buf = NULL;
            }
        }
    }
    fclose(fp);
    return buf;
}

int main(int argc, char** argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s image batch input output\n", argv[0]);
        return 2;
    }
    const int64_t batch = atol(argv[2]);
    long img_len = 0, in_len = 0;
    void* img = read_file(argv[1], &img_len);
    float* host_x = (float*)read_file(argv[3], &in_len);
    if (!img || !host_x) {
        fprintf(stderr, "cannot read the image or the input\n");
        return 1;
    }

    /* tables: check on the host, then one copy into caller memory */
    fcqt_image_info info;
    FCQT(fcqt_image_check(img, img_len, &info));
    void* dtab = NULL;
    HIPCHECK(hipMalloc(&dtab, (size_t)info.device_bytes));
    fcqt_engine_tables et;
    FCQT(fcqt_tables_upload(img, img_len, dtab, info.device_bytes, 0, &et));

    /* buffers, sized by the library */
    fcqt_sizes sz;
    FCQT(fcqt_workspace_sizes(&et.tab, batch, &sz));
    if (in_len != sz.signal) {
        fprintf(stderr, "input has %ld bytes, batch %ld needs %ld\n", in_len, (long)batch, (long)sz.signal);
        return 1;
    }
    float *x, *y, *xs, *work, *f, *kr, *ki;
    HIPCHECK(hipMalloc((void**)&x, (size_t)sz.signal));
    HIPCHECK(hipMalloc((void**)&y, (size_t)sz.signal));
    HIPCHECK(hipMalloc((void**)&xs, (size_t)sz.spectrum));
    HIPCHECK(hipMalloc((void**)&work, (size_t)sz.work));
    HIPCHECK(hipMalloc((void**)&f, (size_t)sz.scatter));
    HIPCHECK(hipMalloc((void**)&kr, (size_t)sz.coef_plane));
    HIPCHECK(hipMalloc((void**)&ki, (size_t)sz.coef_plane));
    FCQT(fcqt_fill_zero(f, sz.scatter / 4, 0)); /* once per F buffer */
    HIPCHECK(hipMemcpy(x, host_x, (size_t)sz.signal, hipMemcpyHostToDevice));

    /* the round trip */
    FCQT(fcqt_analysis(&et.tab, et.route, x, kr, ki, FCQT_PLANAR, xs, work, batch, 0));
    FCQT(fcqt_synthesis(&et.tab, et.scat, et.ovf_scat, kr, ki, FCQT_PLANAR, f, work, y, batch, 0));
    HIPCHECK(hipDeviceSynchronize());

    float* host_y = (float*)malloc((size_t)sz.signal);
    float* host_k = (float*)malloc(2 * (size_t)sz.coef_plane);
    if (!host_y || !host_k) return 1;
    HIPCHECK(hipMemcpy(host_y, y, (size_t)sz.signal, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(host_k, kr, (size_t)sz.coef_plane, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy((char*)host_k + sz.coef_plane, ki, (size_t)sz.coef_plane, hipMemcpyDeviceToHost));
    const int64_t n = sz.signal / 4 / batch;
    for (int64_t b = 0; b < batch; ++b) {
        double num = 0.0, den = 0.0;
        for (int64_t i = 0; i < n; ++i) {
            const double r = host_x[b * n + i], d = r - host_y[b * n + i];
            num += r * r;
            den += d * d;
        }
        printf("row %ld snr %.2f dB\n", (long)b, 10.0 * log10(num / den));
    }
    FILE* out = fopen(argv[4], "wb");
    if (!out || fwrite(host_k, 1, 2 * (size_t)sz.coef_plane, out) != 2 * (size_t)sz.coef_plane) {
        fprintf(stderr, "cannot write %s\n", argv[4]);
        return 1;
    }
    fclose(out);

    /* the single-launch directions on the same buffers: same bits */
    uint32_t* sync;
    HIPCHECK(hipMalloc((void**)&sync, (size_t)sz.sync));
    FCQT(fcqt_fill_zero((float*)sync, sz.sync / 4, 0));
    FCQT(fcqt_persist_analysis(&et.tab, et.route, x, kr, ki, FCQT_PLANAR, xs, work, sync, batch, 0));
    FCQT(fcqt_persist_synthesis(&et.tab, et.scat, et.ovf_scat, kr, ki, FCQT_PLANAR, f, work, y, sync, batch, 0));
    HIPCHECK(hipDeviceSynchronize());
    float* host_y2 = (float*)malloc((size_t)sz.signal);
    float* host_k2 = (float*)malloc(2 * (size_t)sz.coef_plane);
    uint32_t* host_sync = (uint32_t*)malloc((size_t)sz.sync);
    if (!host_y2 || !host_k2 || !host_sync) return 1;
    HIPCHECK(hipMemcpy(host_y2, y, (size_t)sz.signal, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(host_k2, kr, (size_t)sz.coef_plane, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy((char*)host_k2 + sz.coef_plane, ki, (size_t)sz.coef_plane, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(host_sync, sync, (size_t)sz.sync, hipMemcpyDeviceToHost));
    int clear = 1;
    for (int64_t i = 0; i < sz.sync / 4; ++i) clear &= host_sync[i] == 0;
    const int same = memcmp(host_y, host_y2, (size_t)sz.signal) == 0 &&
                     memcmp(host_k, host_k2, 2 * (size_t)sz.coef_plane) == 0;
    printf("single launch: same bits %d, counters and error word clear %d\n", same, clear);
    if (!same || !clear) return 1;
    HIPCHECK(hipFree(sync));
    free(host_y2);
    free(host_k2);
    free(host_sync);

    HIPCHECK(hipFree(x));
    HIPCHECK(hipFree(y));
    HIPCHECK(hipFree(xs));
    HIPCHECK(hipFree(work));
    HIPCHECK(hipFree(f));
    HIPCHECK(hipFree(kr));
    HIPCHECK(hipFree(ki));
    HIPCHECK(hipFree(dtab));
    free(img);
    free(host_x);
    free(host_y);
    free(host_k);
    printf("c round trip ok (batch %ld, ncoef %ld)\n", (long)batch, (long)info.ncoef);
    return 0;
}
