"""CPU oracle for the torch_spyre MI355X hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import anything from here, and only as the
checker (or the timed CPU baseline), never as the measured or shipped path.
The product (torch-spyre_amd/) never imports it.

Contents
  layout.c / layout.py  stick-layout arithmetic (SpyreTensorLayout, allocation
                        sizing, the stick permutation), plain C via ctypes
  ops.py                numpy restatements of the floating-point ops the
                        reference's tests compare against PyTorch CPU
  build.py              compiles layout.c into oracle/_build/liboracle.so

Every function names the reference file:line it follows and the tests in
tests/test_oracle.py pin it (golden vectors, closed forms, brute force).
"""
