"""Layer definitions the native library is compiled for.

The kernels take the hidden size H, the expert intermediate size I, the
number of local experts and the routing parameters (global experts, groups,
groups kept, experts per token) as compile-time constants, as the reference
hard-codes them (kernel.py:615-625) and as its routing kernel takes them as
constexpr parameters (kernel.py:371-389); each definition gets its own
library. The 128-element scale blocks are fixed.

Supported: H a multiple of 1024, I a multiple of 256, 16 / 32 / 64 local
experts, 64 / 128 / 256 global experts in groups of 2 to 16 lanes' worth
(group size / (global experts / 64) in {2, 4, 8, 16}), top_k <= 8, and a
shard whose weights (local experts x 2I x H bytes of gemm1_weights) stay
under 2^31 bytes: the LDS-tiled GEMMs address weight rows with 32-bit
signed offsets.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Definition:
    H: int
    I: int
    EL: int = 32     # local experts of the shard
    EG: int = 256    # global experts
    NG: int = 8      # routing groups
    KG: int = 4      # groups kept per token
    TOPK: int = 8    # experts per token

    @property
    def name(self) -> str:
        g = "" if self.EG == 256 else f"_g{self.EG}"
        return (f"moe_fp8_block_scale_ds_routing_topk{self.TOPK}_ng{self.NG}_kg{self.KG}"
                f"_e{self.EL}{g}_h{self.H}_i{self.I}")

    @property
    def default_routing(self) -> bool:
        return (self.EL, self.EG, self.NG, self.KG, self.TOPK) == (32, 256, 8, 4, 8)

    def defines(self) -> list:
        return [f"-DMI_MOE_HIDDEN={self.H}", f"-DMI_MOE_INTER={self.I}",
                f"-DMI_MOE_E_LOCAL={self.EL}", f"-DMI_MOE_E_GLOBAL={self.EG}",
                f"-DMI_MOE_N_GROUP={self.NG}", f"-DMI_MOE_TOPK_GROUP={self.KG}",
                f"-DMI_MOE_TOP_K={self.TOPK}"]

    @property
    def tag(self) -> str:
        """Build-directory name."""
        return (f"h{self.H}_i{self.I}" if self.default_routing else
                f"h{self.H}_i{self.I}_e{self.EL}_g{self.EG}_ng{self.NG}_kg{self.KG}_k{self.TOPK}")


# moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048
DEFAULT = Definition(7168, 2048)
DEFAULT_SHAPE = (DEFAULT.H, DEFAULT.I)
DEFINITIONS = (
    DEFAULT,
    Definition(4096, 1536),
    # the same layer sharded over 4 GPUs: 64 local experts
    Definition(7168, 2048, EL=64),
    # another routing family: 128 experts in 8 groups of 16, top-3 groups, top-6
    Definition(4096, 1536, EL=16, EG=128, NG=8, KG=3, TOPK=6),
)
# (H, I) of the definitions with the default routing and 32 local experts
SHAPES = tuple((d.H, d.I) for d in DEFINITIONS if d.default_routing)


def supported(H: int, I: int) -> bool:
    return H > 0 and I > 0 and H % 1024 == 0 and I % 256 == 0


def definition_supported(d: Definition) -> bool:
    if not supported(d.H, d.I) or d.EL not in (16, 32, 64) or d.EG not in (64, 128, 256):
        return False
    if d.EG % d.NG:
        return False
    lpg = (d.EG // d.NG) // (d.EG // 64)
    return (lpg in (2, 4, 8, 16) and 1 <= d.KG <= d.NG and 1 <= d.TOPK <= 8
            and d.TOPK <= d.KG * (d.EG // d.NG) and d.EL * 2 * d.I * d.H < (1 << 31))


def as_definition(x) -> Definition:
    """A Definition from a Definition or an (H, I) pair (default routing)."""
    if isinstance(x, Definition):
        return x
    H, I = int(x[0]), int(x[1])
    return Definition(H, I)


def lib_name_of(d: Definition) -> str:
    if d == DEFAULT:
        return "libmi_moe.so"
    return f"libmi_moe_{d.tag}.so"


def lib_name(H: int, I: int) -> str:
    return lib_name_of(Definition(H, I))
