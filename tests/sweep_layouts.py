"""OctCQT layouts beyond the fixture ones, for engine-against-oracle sweeps:
(num_octs, bins_per_oct, fs), every band length in 32..2048. Drawn from the
space of 1-3 octave groups, 4-12 octaves and 4-128 bins per octave at sample
rates of 22.05-192 kHz; several fill a fold list past 200 entries. The
oracle is pinned to the reference on the headline and fixture layouts; here
it is the checker of the engine."""

SWEEP = (
    ([1, 1, 4], [24, 64, 96], 44100),
    ([4, 1, 3], [16, 64, 64], 44100),
    ([3, 2, 4], [4, 4, 24], 44100),
    ([5, 5], [4, 64], 44100),
    ([2, 1, 2], [12, 96, 96], 44100),
    ([5, 2, 1], [4, 16, 24], 48000),
    ([4, 1], [12, 24], 22050),
    ([5, 2, 2], [6, 6, 24], 96000),
    ([4, 3, 1], [12, 12, 24], 192000),
    ([2, 2, 1], [6, 16, 24], 44100),
    ([3, 3, 3], [8, 16, 48], 32000),
)
