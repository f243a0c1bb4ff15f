"""Engine harness around the HIP attention path: a Llama decoder over the flat paged-KV
batch (src/kvserve/model.py of the reference), the KV pool and step execution of its
ModelRunner (src/kvserve/model_runner.py) and HIP-graph decode replay (src/kvserve/
cuda_graph.py). It exists to drive the attention backend the way kvserve does: greedy
token identity against a torch attention backend and decode tokens/s.

Scheduling, prefix caching, sampling beyond greedy, speculative decoding and serving are
kvserve's control plane and are not reproduced here.
"""

from kvserve_amd.engine.config import LLAMA_3_1_8B, LLAMA_3_2_1B, ModelConfig
from kvserve_amd.engine.model import LlamaForCausalLM
from kvserve_amd.engine.runner import DecodeGraphRunner, ModelRunner

__all__ = ["LLAMA_3_1_8B", "LLAMA_3_2_1B", "DecodeGraphRunner", "LlamaForCausalLM", "ModelConfig", "ModelRunner"]
