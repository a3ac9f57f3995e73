"""Drop-in candidates for the reference's ``fastkernels/tasks/candidate`` slot.

``L1/<stem>.py`` defines the class named like the baseline operator in
``fastkernels/tasks/baseline/L1/<stem>.py`` with the same ``__init__`` and
``forward`` signatures, backed by the gfx950 kernels of ``fastkernels_amd``.
"""
