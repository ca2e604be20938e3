"""smel — the MoE-layer hot path of SMEL FT (sparse-MoE LoRA fine-tuning) on MI355X (gfx950) HIP kernels.

Modules mirror the reference's: ``smel.moe`` (router, dispatch, experts, combine, layer), ``smel.lora`` (LoRA
parameter types), ``smel.quant`` (int4 format, int8 head rows), ``smel.pack`` (the packed-layer format, LoRA
merging), ``smel.norm`` (the RMSNorm family around the block), ``smel.stream`` (layer weight streaming),
``smel.loss`` (chunked cross-entropy). Compute runs in
``libsmel_moe.so`` (C-ABI in include/smel_moe.h, smel_norm.h, smel_stream.h and smel_loss.h).
"""
