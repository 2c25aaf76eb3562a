"""CPU oracle for the FP8 linear-layer path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or, for ``cpu_baseline``, as the timed CPU restatement). The product
path in ``jeeves_amd`` never imports it and has no CPU fallback.

The package restates, in numpy, the arithmetic of the reference's FP8 path:

* ``quantize_rows`` (``inference/fp8_weights.py:16-19``) applied to weight rows
  and to token rows of the activations;
* the OCP e4m3fn encode/decode that ``torch.float8_e4m3fn`` implements;
* the exact FP8 x FP8 GEMM (``inference/cuda_test.py:87``), the
  dequantize-then-matmul product, and the reference's W8A16 math
  (``model/metal_test.py:213``);
* the LoRA (``model/lora.py:122-133``) and SwiGLU (``model/model.py:581-584``)
  epilogue formulas;
* the acceptance criteria of ``inference/cuda_test.py:86-93`` and
  ``model/metal_test.py:213-221``.

How each function is pinned is written in its docstring.
"""

from .fp8_ref import *  # noqa: F401,F403
from .fp8_ref import __all__  # noqa: F401
