"""MI355X-native OSCAR INT2 KV-cache hot path (gfx950 HIP kernels behind the reference API).

Modules mirror the reference plugin ``oscar_ascend``: ``config`` (OscarConfig, split/grid
policy), ``layout`` (CacheLayout byte geometry), ``kernels`` (the entry points), plus
``metadata`` (fixed-pointer device metadata) and ``backend`` (the per-layer launch order).
"""

__version__ = "0.1.0"
