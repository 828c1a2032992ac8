"""Training-step pieces around the rasterizer, on the HIP library: the loss
(``loss``), the fused Adam step and clamps (``optim``)."""
