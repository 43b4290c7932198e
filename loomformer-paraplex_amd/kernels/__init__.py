"""Drop-in replacement for the reference's ``kernels`` package on MI355X.

The reference (kernels/build.py:262) JIT-builds one CUDA extension per op
group and returns its pybind module; loomformer.py and tria.py call
``kernels.build.build_or_load(ext_name, sources, ...)`` and then the module's
functions by name.  Here ``build_or_load`` returns a module object with the
same function names, backed by the prebuilt gfx950 library libloom_hip.so.
See ``kernels.build``.
"""
