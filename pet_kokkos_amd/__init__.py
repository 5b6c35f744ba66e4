"""MI355X-native (gfx950 HIP) PET neighbourhood attention, forward and backward.

The product is the C-ABI library ``libpet_attn.so`` (declared in
``include/pet_attn.h``); this package builds it, binds it (``_lib``), mirrors
the reference's ``attention()`` / ``attention_bwd()`` over torch device tensors
(``attention``) and makes the seeded inputs of the benchmark configurations
(``systems``).
"""
