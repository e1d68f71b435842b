"""SGLang-Diffusion attention backend over the Token2Tile MI355X operator."""
