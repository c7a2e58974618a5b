"""CPU oracle for the q4_0 linear and the SDPA default path.

TEST INFRASTRUCTURE ONLY. Only tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker: nothing in ``torchnative_amd`` imports it, and the product path fails
loudly when its HIP library is missing rather than falling back here.

Two layers:

* ``libtnref.so`` (``tnref.c``): a C restatement of the reference's x86_64
  arithmetic, bit for bit where the reference's arithmetic is fully specified
  (codecs, ``vec_dot_unopt``, the matmul driver) and to tolerance where it
  depends on a third-party summation order (SDPA's two GEMMs, the ``gemm``
  crate 0.19.0; "parity unpinned" bitwise).
* ``closed_forms`` (numpy, this package): independent derivations used to pin
  the C restatement -- the exact dyadic value of a quantised matmul, the
  counted Higham bound, an fp64 brute-force attention.
"""

from .oracle import *  # noqa: F401,F403
from .oracle import __all__  # noqa: F401
