"""LoRA-MLP on MI355X (drop-in for kernels/lora_mlp/experiments/{v3,v6})."""
