"""Custom ops of the MoE graph seam (router | stage | MLP)."""
