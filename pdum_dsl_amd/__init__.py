"""pdum_dsl_amd — an MI355X (gfx950) execution backend for the kernels the
pdum.dsl fusion templates produce.

  kernels   device-resident entry points (torch tensors -> libpdhip C ABI)
  tl        the host mirror of the reference's planning interface: IR,
            fusion templates, launch/prune plans, certificates
  hip_tile  compile_tile_hip(region, launch, prune) -> run, the seat of the
            reference's Triton runner
"""

__version__ = "0.1.0"
