from .moe import MoELayer, OffloadMoELayer, TopK, make_moe_layer

__all__ = ["MoELayer", "OffloadMoELayer", "TopK", "make_moe_layer"]
