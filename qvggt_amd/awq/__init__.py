from .qmodule import WQLinear, ScaledActivation, calculate_zeros_width, make_divisible, pack_intweight

__all__ = ["WQLinear", "ScaledActivation", "calculate_zeros_width", "make_divisible", "pack_intweight"]
