"""Parity oracle for the split-manifold LUT path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` (as the checker) and
``bench.py``'s ``cpu_baseline`` leg may import this package.  The product
library never calls into it.

* ``oracle.cpu``          ctypes binding of ``liblut_oracle.so`` (the C
                          restatement of the reference CPU engine)
* ``oracle.ref``          ctypes binding of ``_ref/libojasx_lut_ref.so`` (the
                          reference engine compiled from its own sources;
                          present only where it was built)
* ``oracle.numpy_oracle`` NumPy restatements of the PyTorch engine, the
                          math-engine LUT GEMM, the codec bit packing and the
                          long-context attention / paged KV semantics
* ``oracle.gen``          seeded synthetic inputs for every benchmark config
"""
