"""Seeded synthetic inputs for the five DF-J benchmark systems.

Every array here is plain numpy float64 on the host; the same arrays feed the HIP path (after a
copy into HBM) and the CPU oracle, so both sides see bit-identical inputs.

Conventions fixed by this module (the benchmark descriptions leave them open):

* one ``numpy.random.Generator(PCG64(seed))`` per system, seeds 0..4 in system order;
* splats are shared over atoms near-equally, the remainder going to the first atoms -- the
  placement rule of ``gs_dft/basis/spectral.py:95-107``;
* splat centre = atom position + N(0, 0.4 Bohr) per axis;
* orientation = N(0,1)^4 normalised to a unit quaternion (w, x, y, z);
* per-axis width sigma ~ exp(U(ln 0.3, ln 3)) Bohr and log-precision l = -ln(2 sigma^2), so the
  precision eigenvalue is 1/(2 sigma^2) and the anisotropy ratio of widths is at most 10;
* the product auxiliary basis uses 4 exponent scales (0.5, 1, 2, 4), so N_aux = 4 M;
* C ~ N(0,1), divided by sqrt(k) for the alkane and the two globules; occupations are 1;
* eps = 1e-7, lam = 1e-8, unique pair mode with weights 2 - delta_ij;
* nuclear charges H = 1, C = 6, O = 8 (small random systems cycle 6, 1, 8 over their atoms).

Geometries (Bohr): CO2 with C at the origin and O at z = +-2.196; eight waters with O on a
2x2x2 cubic lattice of spacing 3.0 jittered by U(-0.3, 0.3), H at 1.81 Bohr and 104.5 degrees in
a random orientation; all-trans C20H42 with C-C 1.54 A and C-H 1.09 A at tetrahedral angles;
spherical globules at 0.9 g/cm^3 filled by random sequential placement with a 1.9 Bohr minimum
separation (100 C + 200 H, and 200 C + 400 H + 100 O).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

BOHR_PER_ANGSTROM = 1.0 / 0.529177210903
AUX_SCALES = (0.5, 1.0, 2.0, 4.0)
_AMU_G = 1.66053906660e-24
_MASS = {"H": 1.008, "C": 12.011, "O": 15.999}


@dataclasses.dataclass(frozen=True)
class System:
    """One synthetic DF-J workload: splat parameters, MO coefficients and run knobs."""

    name: str
    atoms: np.ndarray          # (n_atoms, 3) Bohr
    quat: np.ndarray           # (M, 4) unit quaternions (w, x, y, z)
    log_scale: np.ndarray      # (M, 3) log precision eigenvalues
    centers: np.ndarray        # (M, 3) Bohr
    C: np.ndarray              # (M, k)
    occ: np.ndarray            # (k,)
    eps: float = 1e-7
    lam: float = 1e-8
    scales: tuple = AUX_SCALES
    unique: bool = True
    charges: np.ndarray | None = None   # (n_atoms,) nuclear charges, in the order of ``atoms``

    @property
    def M(self) -> int:
        return int(self.centers.shape[0])

    @property
    def k(self) -> int:
        return int(self.C.shape[1])

    @property
    def n_aux(self) -> int:
        return len(self.scales) * self.M


def _splats(atoms: np.ndarray, M: int, rng: np.random.Generator):
    n_atoms = atoms.shape[0]
    base, rem = divmod(M, n_atoms)
    counts = [base + (1 if a < rem else 0) for a in range(n_atoms)]
    centers = np.repeat(atoms, counts, axis=0) + rng.normal(0.0, 0.4, (M, 3))
    q = rng.normal(size=(M, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    sigma = np.exp(rng.uniform(math.log(0.3), math.log(3.0), (M, 3)))
    log_scale = -np.log(2.0 * sigma * sigma)
    return q, log_scale, centers


def _random_rotation(rng: np.random.Generator) -> np.ndarray:
    q = rng.normal(size=4)
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def co2_atoms() -> np.ndarray:
    return np.array([[0.0, 0.0, 0.0], [0.0, 0.0, 2.196], [0.0, 0.0, -2.196]])


def water_octamer_atoms(rng: np.random.Generator) -> np.ndarray:
    r_oh, half = 1.81, math.radians(104.5) / 2.0
    local_h = np.array([[r_oh * math.sin(half), 0.0, r_oh * math.cos(half)],
                        [-r_oh * math.sin(half), 0.0, r_oh * math.cos(half)]])
    out = []
    for ix in range(2):
        for iy in range(2):
            for iz in range(2):
                o = 3.0 * np.array([ix, iy, iz], float) + rng.uniform(-0.3, 0.3, 3)
                R = _random_rotation(rng)
                out.append(o)
                out.extend(o + local_h @ R.T)
    return np.array(out)


def alkane_atoms(n_carbon: int = 20) -> np.ndarray:
    """All-trans CnH(2n+2): zig-zag backbone in the xz plane, tetrahedral hydrogens."""
    cc, ch = 1.54 * BOHR_PER_ANGSTROM, 1.09 * BOHR_PER_ANGSTROM
    tet = math.acos(-1.0 / 3.0)
    dx, dz = cc * math.sin(tet / 2.0), cc * math.cos(tet / 2.0)
    carbons = np.array([[i * dx, 0.0, (dz if i % 2 else 0.0)] for i in range(n_carbon)])
    hyd = []
    for i, c in enumerate(carbons):
        nbrs = [carbons[j] for j in (i - 1, i + 1) if 0 <= j < n_carbon]
        if len(nbrs) == 1:                            # chain end: extend the zig-zag
            prev = nbrs[0]
            nbrs.append(c + (c - prev) * np.array([1.0, 1.0, -1.0]))
        u1 = (nbrs[0] - c) / np.linalg.norm(nbrs[0] - c)
        u2 = (nbrs[1] - c) / np.linalg.norm(nbrs[1] - c)
        bis = -(u1 + u2) / np.linalg.norm(u1 + u2)
        perp = np.cross(u1, u2) / np.linalg.norm(np.cross(u1, u2))
        half = tet / 2.0
        dirs = [math.cos(half) * bis + math.sin(half) * perp,
                math.cos(half) * bis - math.sin(half) * perp]
        if i in (0, n_carbon - 1):                    # methyl: the virtual neighbour is an H
            dirs.append((nbrs[1] - c) / np.linalg.norm(nbrs[1] - c))
        hyd.extend(c + ch * d for d in dirs)
    return np.concatenate([carbons, np.array(hyd)])


def globule_atoms(counts: dict, rng: np.random.Generator, density: float = 0.9,
                  min_sep: float = 1.9) -> np.ndarray:
    """Random sequential placement in a sphere whose volume gives ``density`` g/cm^3."""
    mass_g = sum(_MASS[e] * c for e, c in counts.items()) * _AMU_G
    vol_a3 = mass_g / density * 1e24
    radius = (3.0 * vol_a3 / (4.0 * math.pi)) ** (1.0 / 3.0) * BOHR_PER_ANGSTROM
    n = sum(counts.values())
    pts = np.empty((n, 3))
    m = 0
    while m < n:
        p = rng.uniform(-radius, radius, 3)
        if p @ p > radius * radius:
            continue
        if m and np.min(np.sum((pts[:m] - p) ** 2, axis=1)) < min_sep * min_sep:
            continue
        pts[m] = p
        m += 1
    return pts


_SPECS = {
    1: ("co2", 126, 11, False),
    2: ("water8", 600, 40, False),
    3: ("c20h42", 2000, 81, True),
    4: ("globule300", 12000, 600, True),
    5: ("globule700", 20000, 1300, True),
}

NAMES = {v[0]: k for k, v in _SPECS.items()}

# Nuclear charges in the order each geometry lists its atoms (globules place the elements of
# their count table in order).
_CHARGES = {
    1: lambda: np.array([6.0, 8.0, 8.0]),
    2: lambda: np.tile([8.0, 1.0, 1.0], 8),
    3: lambda: np.array([6.0] * 20 + [1.0] * 42),
    4: lambda: np.array([6.0] * 100 + [1.0] * 200),
    5: lambda: np.array([6.0] * 200 + [1.0] * 400 + [8.0] * 100),
}


def make_system(index: int, *, eps: float = 1e-7) -> System:
    """Benchmark system ``index`` in 1..5 (seed ``index - 1``)."""
    if index not in _SPECS:
        raise ValueError(f"system index must be one of {sorted(_SPECS)}, got {index}")
    name, M, k, scale_c = _SPECS[index]
    rng = np.random.Generator(np.random.PCG64(index - 1))
    if index == 1:
        atoms = co2_atoms()
    elif index == 2:
        atoms = water_octamer_atoms(rng)
    elif index == 3:
        atoms = alkane_atoms(20)
    elif index == 4:
        atoms = globule_atoms({"C": 100, "H": 200}, rng)
    else:
        atoms = globule_atoms({"C": 200, "H": 400, "O": 100}, rng)
    quat, log_scale, centers = _splats(atoms, M, rng)
    C = rng.normal(size=(M, k))
    if scale_c:
        C /= math.sqrt(k)
    return System(name=name, atoms=atoms, quat=quat, log_scale=log_scale, centers=centers,
                  C=C, occ=np.ones(k), eps=eps, charges=_CHARGES[index]())


def make_globule2100(k: int = 16, eps: float = 1e-7) -> System:
    """A screening-scale shape beyond the benchmark systems: a 2100-atom C/H/O globule (600 C,
    1200 H, 300 O) at 0.9 g/cm^3 with M = 60000 splats (seed 5), the per-GPU splat count of the
    reference's largest size-ladder runs. Only its pair list is built at this size, so C has a
    few columns."""
    rng = np.random.Generator(np.random.PCG64(5))
    atoms = globule_atoms({"C": 600, "H": 1200, "O": 300}, rng)
    M = 60000
    quat, log_scale, centers = _splats(atoms, M, rng)
    C = rng.normal(size=(M, k)) / math.sqrt(k)
    return System(name="globule2100", atoms=atoms, quat=quat, log_scale=log_scale,
                  centers=centers, C=C, occ=np.ones(k), eps=eps,
                  charges=np.array([6.0] * 600 + [1.0] * 1200 + [8.0] * 300))


def make_small(M: int, k: int, n_atoms: int = 4, seed: int = 0, spread: float = 2.5,
               width=(0.3, 3.0), n_scales: int = 2) -> System:
    """A small random system for parity tests: ``n_atoms`` random atoms in a cube of half-side
    ``spread`` Bohr, splats placed by the same rule as the benchmark systems."""
    rng = np.random.Generator(np.random.PCG64(1000 + seed))
    atoms = rng.uniform(-spread, spread, (n_atoms, 3))
    n = M
    base, rem = divmod(n, n_atoms)
    counts = [base + (1 if a < rem else 0) for a in range(n_atoms)]
    centers = np.repeat(atoms, counts, axis=0) + rng.normal(0.0, 0.4, (M, 3))
    q = rng.normal(size=(M, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    sigma = np.exp(rng.uniform(math.log(width[0]), math.log(width[1]), (M, 3)))
    log_scale = -np.log(2.0 * sigma * sigma)
    C = rng.normal(size=(M, k)) / math.sqrt(k)
    scales = AUX_SCALES[1:1 + n_scales] if n_scales < len(AUX_SCALES) else AUX_SCALES
    return System(name=f"small{M}", atoms=atoms, quat=q, log_scale=log_scale, centers=centers,
                  C=C, occ=np.ones(k), scales=tuple(scales),
                  charges=np.resize(np.array([6.0, 1.0, 8.0]), n_atoms))


def atom_grid(atoms: np.ndarray, n_rad: int = 24, n_ang: int = 110, r_max: float = 12.0,
              seed: int = 0) -> np.ndarray:
    """Synthetic atom-centred grid points (Bohr) for the density-on-grid workloads: per atom,
    ``n_rad`` radii on a log-spaced ladder up to ``r_max`` times ``n_ang`` directions of a
    Fibonacci sphere, randomly rotated per atom. Points only (the density needs no weights)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    radii = r_max * (np.expm1(np.linspace(0.05, 3.0, n_rad)) / np.expm1(3.0))
    i = np.arange(n_ang) + 0.5
    phi = np.arccos(1.0 - 2.0 * i / n_ang)
    th = math.pi * (1.0 + 5.0 ** 0.5) * i
    dirs = np.stack([np.cos(th) * np.sin(phi), np.sin(th) * np.sin(phi), np.cos(phi)], axis=1)
    out = []
    for a in atoms:
        R = _random_rotation(rng)
        out.append(a + (radii[:, None, None] * (dirs @ R.T)[None, :, :]).reshape(-1, 3))
    return np.concatenate(out)

