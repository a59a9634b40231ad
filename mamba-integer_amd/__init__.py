"""MI355X-native integer Mamba inference path.

Put this directory on sys.path (as the reference does with its src/) to use
the drop-in modules ``mamba_integer_model`` and ``rational_bitnet``; the
implementation package is ``mamba_int``.
"""
