"""MI355X-native ALoDLM training step: Python host code over gfx950 HIP kernels.

Module names mirror the reference package ``alodlm`` (config, batch, attention,
model, train) so that ``import alodlm_amd as alodlm`` is the drop-in.
"""

__version__ = "0.1.0"
