"""The MI355X device spec, in the reference's device-spec format.

`QuailBackend.supports` admits only devices listed in
quail/specs/data/devices/*.toml (quail/backends/quail/backend.py:28-30),
each a `DeviceSpec` (quail/specs/base.py:404-436). `devices/mi355x.toml`
here is that file for the MI355X; `read_device` parses it with the same
field set and the same positivity check, so it can be dropped into the
reference's devices folder as it is.
"""

from dataclasses import dataclass, fields
from pathlib import Path

DEVICES = Path(__file__).resolve().parent / "devices"


@dataclass(frozen=True)
class DeviceSpec:
    name: str
    mem_bytes: float
    hbm_bw: float
    fp8_flops: float
    bf16_flops: float
    fp32_flops: float
    usd_per_hour: float = 0.0
    price_source: str = ""
    cuda_name: str = ""
    modal_gpu: str = ""
    page_tokens: int = 16
    mamf_fp8_flops: float = 0.0
    mamf_bf16_flops: float = 0.0
    fp4_flops: float = 0.0

    def __post_init__(self):
        for precision in ("fp8", "bf16", "fp32"):
            if not getattr(self, f"{precision}_flops") > 0:
                raise ValueError(f"{self.name}: {precision}_flops must be positive")


def read_device(path) -> DeviceSpec:
    """Parse one device TOML; its file name must be its spec's name.

    Raises:
        ValueError: a key that is not a DeviceSpec field, or a name mismatch.
    """
    try:
        import tomllib
    except ModuleNotFoundError:  # Python 3.10
        import tomli as tomllib
    path = Path(path)
    with open(path, "rb") as f:
        data = tomllib.load(f)
    known = {f.name for f in fields(DeviceSpec)}
    unknown = set(data) - known
    if unknown:
        raise ValueError(f"{path.name}: unknown keys {sorted(unknown)}")
    spec = DeviceSpec(**data)
    if spec.name != path.stem:
        raise ValueError(f"{path.name}: spec name {spec.name!r} differs from the file name")
    return spec


MI355X = read_device(DEVICES / "mi355x.toml")
