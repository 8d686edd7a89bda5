"""cliffordcuda_amd: Clifford algebra Cl(p, q, r) products, rotors and graded
ops on AMD MI355X (gfx950), drop-in for the ``cliffordcuda`` API.

Same public names as the reference package (``src/cliffordcuda/__init__.py``),
plus ``left_contraction`` / ``right_contraction`` spellings.
"""
from .algebra import CliffordAlgebra
from .products import (
    geom_prod, geom_prod_multik,
    wedge_prod, wedge_prod_multik, wedge_prod_skip, wedge_prod_multik_skip, wedge_prod_subset_grade,
    inner_prod, inner_prod_kskip, inner_prod_multik, inner_prod_multik_skip, inner_prod_skip,
    inner_prod_subset_grade,
    left_contract, left_contract_skip, left_contract_subset_grade,
    right_contract, right_contract_skip, right_contract_subset_grade,
    left_contraction, right_contraction,
    regressive_prod, regressive_prod_skip, regressive_prod_subset_grade,
)
from .graded import reverse
from .inverse import inverse
from .layers import (
    GeometricProductLayer, WedgeProductLayer, InnerProductLayer,
    LeftContractionLayer, RightContractionLayer, RegressiveProductLayer,
    RotorLayer,
)

__all__ = [
    "CliffordAlgebra",
    "geom_prod", "geom_prod_multik",
    "wedge_prod", "wedge_prod_multik", "wedge_prod_skip",
    "wedge_prod_multik_skip", "wedge_prod_subset_grade",
    "inner_prod", "inner_prod_kskip", "inner_prod_multik",
    "inner_prod_multik_skip", "inner_prod_skip", "inner_prod_subset_grade",
    "left_contract", "left_contract_skip", "left_contract_subset_grade",
    "right_contract", "right_contract_skip", "right_contract_subset_grade",
    "left_contraction", "right_contraction",
    "regressive_prod", "regressive_prod_skip", "regressive_prod_subset_grade",
    "inverse", "reverse",
    "GeometricProductLayer", "WedgeProductLayer", "InnerProductLayer",
    "LeftContractionLayer", "RightContractionLayer", "RegressiveProductLayer",
    "RotorLayer",
]
__version__ = "0.1.0"
