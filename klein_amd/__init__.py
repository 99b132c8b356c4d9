"""MI355X (gfx950) implementation of klein's token-sampling path: penalties, temperature, top-k, softmax,
min-p/top-p, the seeded draw (src/sampler.cpp) and the MTP verify accept rule (src/engine.cpp:563-575), as HIP
kernels behind the C ABI of include/klein_sampler.h."""
from .workloads import Params, VOCAB  # noqa: F401
from .sampler import Sampler, debug_expf, debug_sum_replay  # noqa: F401
from . import _lib  # noqa: F401


def library_path() -> str:
    return _lib.LIB_PATH
