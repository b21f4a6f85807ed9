"""Packaging for the MI355X Q8_0 paged-attention vLLM plugin.

Same distribution surface as the reference (``extension/setup.py:52-60``):
top-level modules ``gfx906_fa_backend`` and ``gfx906_fa_paged`` plus the op
module ``gfx906_fa``, and the vLLM entry point
``vllm.general_plugins: gfx906_fa = gfx906_fa_backend:register``.
The HIP library is built by ``build.py`` (hipcc, gfx950) and shipped next to
the modules.

    python build.py && pip install -e .
"""
from setuptools import setup
from setuptools.command.build_py import build_py


class _BuildHip(build_py):
    def run(self):
        import build as _b  # noqa: PLC0415  (local build.py)
        _b.build(verbose=True)
        super().run()


setup(
    name="gfx906_fa_amd",
    version="0.1.0",
    py_modules=["gfx906_fa", "gfx906_fa_backend", "gfx906_fa_paged"],
    data_files=[("", ["libgfx906_fa_amd.so"])],
    entry_points={
        "vllm.general_plugins": [
            "gfx906_fa = gfx906_fa_backend:register",
        ],
    },
    cmdclass={"build_py": _BuildHip},
)
