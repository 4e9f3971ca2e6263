"""MI355X-native routed-MoE layer for livglm's GLM-5.3-Flash.

Host-side mirror of the reference's MoE interface (``moe.py``, ``expert_ssd.py``,
``layers.py``), of the decoder FFN site around it (``mhc.py``, ``model.py``) and
of its checkpoint side (the safetensors index, the bank load plan, ScaleX
scale coding and layer containers) on torch tensors, computed by the HIP library
``libglm53moe.so`` (``livglm_amd``).  Every expert is resident in HBM.
"""

__all__ = [
    "bank_loader",
    "bank_plan",
    "checkpoint",
    "contract",
    "expert_ssd",
    "layers",
    "mhc",
    "model",
    "model_config",
    "moe",
    "scale_codec",
    "scalex_layer",
]
