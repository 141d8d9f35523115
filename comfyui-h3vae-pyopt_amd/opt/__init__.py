"""Host-side mirror of the reference's hot-path operator modules.

Each module keeps the reference module's name, public functions and
``torch.library`` op names (fishelegs/ComfyUI-H3VAE-PyOpt ``opt/*.py``), and
runs the arithmetic on the gfx950 kernels of ``libh3vae_hip.so``.
"""
