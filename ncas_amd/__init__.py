"""MI355X-native NCA step / rollout engine.

The compute runs in `libnca_hip.so` (hand-written HIP for gfx950, C ABI in include/nca_hip.h);
this package is the host side that mirrors the reference engine's interfaces:

* `model`     - NCAConfig / NCA parameter container (reference src/nca/model.py names)
* `step`      - make_step / StepOptions: the per-step drop-in (reference engine/step.py)
* `inference` - rollout_steps (fused multi-step op) and InferenceEngine (engine/inference.py)
* `rollout`   - rollout / conf_at_k / pass_at_k / select_at_k (reference rollout.py)
* `readout`   - confidence, decode, conf@K selection on the GPU
* `rng`       - Philox fire masks
* `tasks`     - Boards and the maze / Sudoku generators
"""

from .model import NCA, NCAConfig, build_model, init_weights  # noqa: F401

__all__ = ["NCA", "NCAConfig", "build_model", "init_weights"]
