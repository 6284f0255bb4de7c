"""Reference-shaped callers of the MoE layer, used to run and measure it in context.

blocks.py   pre-norm RMSNorm -> MoE -> residual block and the 12-block stack
            (lib/blocks/encoder.py:73-90 without attention)
encoder.py  GeneT5-shaped encoder with ALiBi attention (the HIP varlen kernel by
            default, the PyTorch SDPA composition on request) and the MoE in every
            layer, plus the MDLM iterative-unmasking driver (config 5;
            lib/model/genet5.py:11-59, lib/inference/diffusion_engine.py:5-95)
"""
