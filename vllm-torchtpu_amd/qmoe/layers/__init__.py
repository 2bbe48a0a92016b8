"""Mirrors of the reference plugin's adapter entry points for the
quantized-matmul / fused-MoE path (`layers/adapter/` of vllm_torchtpu)."""
