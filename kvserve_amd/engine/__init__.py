"""Engine harness around the HIP attention path: a Llama decoder over the flat paged-KV
batch (the model of src/kvserve/model.py in the reference), its KV pool, step execution with
kvserve's three paths (decode graph, piecewise graphs around eager attention, eager;
src/kvserve/model_runner.py, src/kvserve/cuda_graph.py) and a scheduler-free batcher that
mixes prefill chunks with decodes. It exists to drive the attention backend the way kvserve
does: greedy token identity against a torch attention backend and decode tokens/s.

Scheduling policy, preemption, prefix caching, sampling beyond greedy, speculative decoding
and serving are kvserve's control plane and are not reproduced here.
"""

from kvserve_amd.engine.config import LLAMA_3_1_8B, LLAMA_3_2_1B, ModelConfig
from kvserve_amd.engine.model import PagedLlama, build_model
from kvserve_amd.engine.runner import Batcher, DecodeGraphRunner, ModelRunner, PiecewiseGraphRunner, Sequence, generate

__all__ = [
    "LLAMA_3_1_8B",
    "LLAMA_3_2_1B",
    "Batcher",
    "DecodeGraphRunner",
    "ModelConfig",
    "ModelRunner",
    "PagedLlama",
    "PiecewiseGraphRunner",
    "Sequence",
    "build_model",
    "generate",
]
