"""CPU oracle for the fused factored CQT hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``flash-cqt_amd/``) may
import, call or execute anything in this package. The only permitted callers
are ``tests/``, ``__graft_entry__.smoke()`` (as the checker of one GPU call)
and the ``cpu_baseline`` leg of ``bench.py`` (as the timed host-core port).

Contents
  cqt_oracle    numpy restatement of the reference transform definition:
                window helpers (ref_util.py), FlexOctBank (filterbank.py),
                OctCQT tables and fwd/bwd (oct_cqt.py), both adjoints
                (trainable.py:111-139 semantics), the packed real FFT
                identities (bench/packedfft.py:73-85) and SlicedCQT
                (sliced.py). Tables are built in float32 exactly as the
                reference builds them; transforms run in float64.
  torch_port    the same transform as torch ops in float32 on the host CPU,
                used as the autograd reference for gradients and as the
                timed host-core baseline.

Pinning (what checks each function, so a plausible mistake fails one):
  bank tables        golden fixtures written by tests/golden/make_golden.py
                     from the reference itself (bit-exact float32 compare)
  fwd / bwd          golden coefficient vectors from the reference; float64
                     perfect reconstruction (painless frame, > 250 dB);
                     linearity; band energy sums
  adjoints           dot-product identity <A x, y> = <x, A^T y> in float64;
                     golden gradient vectors from reference autograd
  packed FFT         numpy.fft on identical inputs (closed form DFT)
  sliced             golden sliced vectors from the reference; stream equals
                     whole buffer; round trip
"""
