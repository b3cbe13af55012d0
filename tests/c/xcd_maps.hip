// Host build of the kernels' own workgroup maps (fcqt_fft.hpp xcd_remap and
// xcd_remap_reverse are __host__ __device__): prints, for each grid size
// given on the command line, the logical id of every dispatch id under both
// maps, one line per grid: "G fwd... | rev...", or with "band NT B" the
// (task, slice) of every logical band workgroup under both band orders
// (band_place). tests/test_tables.py compares these with the simulator's
// replicas.
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../flash-cqt_amd/csrc/fcqt_fft.hpp"

int main(int argc, char** argv) {
    // "band NT B": band_place of every logical id of an NT x B band grid,
    // task-major then slice-major, one line each: "task,b ..."
    if (argc == 4 && std::string(argv[1]) == "band") {
        const int nt = std::atoi(argv[2]), batch = std::atoi(argv[3]);
        for (int order = 0; order < 2; ++order) {
            for (int lg = 0; lg < nt * batch; ++lg) {
                int task = -1, b = -1;
                fcqt::band_place(lg, nt, batch, order != 0, task, b);
                std::printf("%s%d,%d", lg ? " " : "", task, b);
            }
            std::printf("\n");
        }
        return 0;
    }
    for (int a = 1; a < argc; ++a) {
        const int G = std::atoi(argv[a]);
        std::printf("%d", G);
        for (int l = 0; l < G; ++l) std::printf(" %d", fcqt::xcd_remap(l, G));
        std::printf(" |");
        for (int l = 0; l < G; ++l) std::printf(" %d", fcqt::xcd_remap_reverse(l, G));
        std::printf("\n");
    }
    return 0;
}
