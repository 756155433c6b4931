"""LoRA-QKV on MI355X (drop-in for kernels/lora_qkv/experiments/{v2,v3,v4})."""
