"""kandiga_amd -- MI355X-native routed-expert MoE layer (MLX 3/4-bit experts, top-K)."""
__version__ = "0.1.0"
