"""tandem_amd: an MI355X-native (gfx950) AWQ W4A16 linear path, drop-in for tandem's layers/awq.py.

    from tandem_amd.layers.awq import W4Linear
"""

__version__ = "0.1.0"
