"""Host-side data preparation for MoE routing replay: vLLM route capture and packing."""
