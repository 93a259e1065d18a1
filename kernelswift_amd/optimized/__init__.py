"""Drop-in ModelNew modules: same constructors, forward signatures, parameter and buffer names as the
reference's optimized/*/ wrappers over baseline/*.py, computed by the gfx950 kernels of libkswift_amd.so.

Each file is self-contained and loads the library lazily inside a function, so an auto_bench-style
harness that keeps only imports, defs, classes and literal assignments of a module can load it by path.
"""
