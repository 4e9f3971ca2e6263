"""MI355X-native routed-MoE layer for livglm's GLM-5.3-Flash.

Host-side mirror of the reference's MoE interface (``moe.py``, ``expert_ssd.py``,
``layers.py``) on torch tensors, computed by the HIP library ``libglm53moe.so``
(``livglm_amd``).  Every expert is resident in HBM.
"""

__all__ = [
    "bank_loader",
    "contract",
    "expert_source",
    "expert_ssd",
    "layers",
    "model_config",
    "moe",
]
