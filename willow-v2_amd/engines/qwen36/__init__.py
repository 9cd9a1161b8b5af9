from .moe_hip import HipMoE  # noqa: F401
