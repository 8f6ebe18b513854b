"""noise_amd: Noise's forward-only population training hot path on MI355X (gfx950) HIP kernels.

Host API mirrors the reference: noise_amd.model (utils/model.py), noise_amd.population (eggroll.py),
noise_amd.credit (the credit readout ops), noise_amd.optim (AdamW on the fused kernel).
"""
from .model import GPT, GPTConfig  # noqa: F401
