// Host build of the kernels' own workgroup maps (fcqt_fft.hpp xcd_remap and
// xcd_remap_reverse are __host__ __device__): prints, for each grid size
// given on the command line, the logical id of every dispatch id under both
// maps, one line per grid: "G fwd... | rev...". tests/test_tables.py compares
// these with the simulator's replicas.
#include <cstdio>
#include <cstdlib>

#include "../../flash-cqt_amd/csrc/fcqt_fft.hpp"

int main(int argc, char** argv) {
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
