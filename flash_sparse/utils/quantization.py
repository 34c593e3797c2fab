"""Reference module path of the quantisation helpers (``flash_sparse/utils/quantization.py``)."""

from streamindex_amd.quant import act_quant, act_quant_simulate, fp4_act_quant, fp4_act_quant_simulate

__all__ = ["act_quant_simulate", "fp4_act_quant_simulate", "act_quant", "fp4_act_quant"]
