"""Seeded synthetic manipulation scenes (the model intake of this backend).

The reference compiles LIBERO MJCF with CPU MuJoCo (``gpu/host/backends/cuda_fp32/scene.py:88-143``)
and preprocesses the compiled model (``gpu/host/backends/cuda_fp32/model.py:30-219``).  MuJoCo is
not part of this backend, so scenes are described here directly, as a tree of bodies carrying
joints, geoms, sites and actuators, in MuJoCo's conventions (quaternions are w,x,y,z; joint types
free=0, slide=2, hinge=3; geom types plane=0, sphere=2, capsule=3, box=6, mesh=7).

Five scene families are produced, one per benchmark configuration:

* ``c1``  arm + table + 3 free boxes, elliptic cones, N=2 (the CPU-runnable case);
* ``c2``  arm only, constraints disabled (smooth dynamics), N=1024;
* ``c3``  arm + table + 2 boxes + 2 capsules + 2 convex hulls, pyramidal cones, mu=1, N=4096;
* ``c4``  arm + table + 20 objects in two layers, N=8192;
* ``c5``  arm + table + 12 object slots of which each world activates U{0..12}, N=16384.

The robot is a 7-revolute serial arm (alternating z/y axes) with a 2-slide gripper, driven by
7 torque motors and 2 finger position servos (nu=9), the actuator set the reference controller
requires (``gpu/host/backends/cuda_fp32/controller.py:46-52``).
"""
from __future__ import annotations

from dataclasses import dataclass, field
import math

import numpy as np

FREE, BALL, SLIDE, HINGE = 0, 1, 2, 3
PLANE, SPHERE, CAPSULE, ELLIPSOID, CYLINDER, BOX, MESH = 0, 2, 3, 4, 5, 6, 7
PYRAMIDAL, ELLIPTIC = 0, 1

# MuJoCo disable bits used by this backend (mjtDisableBit).
DISABLE_CONSTRAINT = 1 << 0
DISABLE_FRICTIONLOSS = 1 << 2
DISABLE_LIMIT = 1 << 3
DISABLE_CONTACT = 1 << 4
DISABLE_PASSIVE = 1 << 5
DISABLE_GRAVITY = 1 << 6
DISABLE_WARMSTART = 1 << 8
DISABLE_ACTUATION = 1 << 10
DISABLE_EULERDAMP = 1 << 15
DISABLE_NATIVECCD = 1 << 17      # box-box by the primitive SAT routine instead of GJK/EPA

SOLREF_DEFAULT = (0.02, 1.0)
SOLIMP_DEFAULT = (0.9, 0.95, 0.001, 0.5, 2.0)


@dataclass
class Joint:
    type: int
    axis: tuple = (0.0, 0.0, 1.0)
    pos: tuple = (0.0, 0.0, 0.0)
    limited: bool = False
    range: tuple = (0.0, 0.0)
    damping: float = 0.0
    armature: float = 0.0
    stiffness: float = 0.0
    springref: float = 0.0
    frictionloss: float = 0.0
    margin: float = 0.0
    solref: tuple = SOLREF_DEFAULT
    solimp: tuple = SOLIMP_DEFAULT
    actuatorgravcomp: bool = False   # gravity compensation of this joint reported as actuator force


@dataclass
class Geom:
    type: int
    size: tuple = (0.0, 0.0, 0.0)
    pos: tuple = (0.0, 0.0, 0.0)
    quat: tuple = (1.0, 0.0, 0.0, 0.0)
    contype: int = 1
    conaffinity: int = 1
    condim: int = 3
    priority: int = 0
    friction: tuple = (1.0, 0.005, 0.0001)
    solref: tuple = SOLREF_DEFAULT
    solimp: tuple = SOLIMP_DEFAULT
    solmix: float = 1.0
    margin: float = 0.0
    gap: float = 0.0
    vertices: np.ndarray | None = None   # convex hull vertices in the geom frame (mesh only)


@dataclass
class Site:
    pos: tuple = (0.0, 0.0, 0.0)
    quat: tuple = (1.0, 0.0, 0.0, 0.0)
    name: str = ''


@dataclass
class Body:
    name: str
    parent: int
    pos: tuple = (0.0, 0.0, 0.0)
    quat: tuple = (1.0, 0.0, 0.0, 0.0)
    mass: float = 0.0
    inertia: tuple = (0.0, 0.0, 0.0)
    ipos: tuple = (0.0, 0.0, 0.0)
    iquat: tuple = (1.0, 0.0, 0.0, 0.0)
    joints: list = field(default_factory=list)
    geoms: list = field(default_factory=list)
    sites: list = field(default_factory=list)
    gravcomp: float = 0.0            # fraction of the body's weight compensated (MuJoCo body gravcomp)


@dataclass
class Sensor:
    kind: str                  # 'force' or 'torque' (MuJoCo sensor types 4 and 5)
    site: int                  # global site index
    cutoff: float = 0.0        # 0: no clipping


@dataclass
class Actuator:
    joint: int                 # global joint index
    kind: str                  # 'motor' or 'position'
    gear: float = 1.0
    kp: float = 0.0
    kv: float = 0.0
    ctrlrange: tuple = (-1.0, 1.0)
    forcerange: tuple = (0.0, 0.0)
    forcelimited: bool = False


@dataclass
class Options:
    timestep: float = 0.002
    gravity: tuple = (0.0, 0.0, -9.81)
    iterations: int = 100
    tolerance: float = 1e-6          # FP32 floor of the reference (gpu/precision.py:79-81)
    ls_iterations: int = 50
    ls_tolerance: float = 0.01
    cone: int = ELLIPTIC
    impratio: float = 20.0           # LIBERO default (gpu/host/runtime/constraints/identity.py:7)
    disableflags: int = 0
    nconmax: int = 64
    njmax: int = 0                   # 0: derived from nconmax and the cone
    ccd_iterations: int = 35         # GJK / EPA iteration cap (MuJoCo opt.ccd_iterations)
    ccd_tolerance: float = 1e-6      # GJK / EPA tolerance (MuJoCo opt.ccd_tolerance)
    density: float = 0.0             # medium density (MuJoCo opt.density; 0: no quadratic drag)
    viscosity: float = 0.0           # medium viscosity (MuJoCo opt.viscosity; 0: no viscous drag)
    wind: tuple = (0.0, 0.0, 0.0)    # medium velocity (MuJoCo opt.wind)
    mpr: bool = False                # MuJoCo 2.3.7 collision semantics: convex pairs by MPR (one contact),
                                     # box-box by the primitive routine
    mpr_iterations: int = 50         # MuJoCo opt.mpr_iterations
    mpr_tolerance: float = 1e-6      # MuJoCo opt.mpr_tolerance


@dataclass
class Scene:
    name: str
    bodies: list
    actuators: list
    options: Options
    nworld: int
    substeps: int
    osc: dict
    init_qpos: np.ndarray            # (nworld, nq) initial states, float64
    init_qvel: np.ndarray            # (nworld, nv)
    body_active: np.ndarray | None = None   # (nworld, nbody) int32, heterogeneous batches only
    seed: int = 0
    sensors: list = field(default_factory=list)


def quat_yaw(angle):
    return (math.cos(angle / 2), 0.0, 0.0, math.sin(angle / 2))


def box_inertia(mass, half):
    a, b, c = (2 * h for h in half)
    return (mass / 12 * (b * b + c * c), mass / 12 * (a * a + c * c), mass / 12 * (a * a + b * b))


def capsule_mass_inertia(density, radius, half_length):
    """Solid capsule along z: cylinder of height 2h plus two hemispheres (MuJoCo's capsule rule)."""
    r, h = radius, half_length
    vcyl = math.pi * r * r * 2 * h
    vhem = 2.0 / 3.0 * math.pi * r ** 3
    mcyl, mhem = density * vcyl, density * vhem
    mass = mcyl + 2 * mhem
    izz = mcyl * r * r / 2 + 2 * mhem * 2 * r * r / 5
    # hemisphere about its own centroid, shifted to the capsule centre
    ih = 83.0 / 320.0 * mhem * r * r
    dist = h + 3.0 * r / 8.0
    ixx = mcyl * (3 * r * r + (2 * h) ** 2) / 12 + 2 * (ih + mhem * dist * dist)
    return mass, (ixx, ixx, izz)


def hull_mass_properties(vertices, density):
    """Volume, centroid and inertia tensor of a convex hull by signed tetrahedra."""
    from scipy.spatial import ConvexHull
    hull = ConvexHull(vertices)
    centre = vertices[hull.vertices].mean(axis=0)
    volume = 0.0
    first = np.zeros(3)
    second = np.zeros((3, 3))
    canon = np.array([[2, 1, 1], [1, 2, 1], [1, 1, 2]], float) / 120.0
    for simplex in hull.simplices:
        a, b, c = vertices[simplex] - centre
        n = np.cross(b - a, c - a)
        if np.dot(n, a) < 0:
            b, c = c, b
        d = np.column_stack([a, b, c])
        det = np.linalg.det(d)
        volume += det / 6.0
        first += det / 24.0 * (a + b + c)
        second += det * d @ canon @ d.T
    com = first / volume + centre
    second_c = second - volume * np.outer(first / volume, first / volume)
    inertia = density * (np.trace(second_c) * np.eye(3) - second_c)
    return density * volume, com, inertia, hull


def make_hull(rng, npoints, semi_axes):
    """Points on a jittered ellipsoid, hulled, recentred on the centroid and aligned with the
    principal axes (the mesh-frame convention MuJoCo uses for mesh geoms)."""
    for _ in range(100):
        dirs = rng.normal(size=(npoints, 3))
        dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
        pts = dirs * np.asarray(semi_axes) * rng.uniform(0.85, 1.0, size=(npoints, 1))
        mass_one, com, inertia, hull = hull_mass_properties(pts, 1.0)
        if len(hull.vertices) >= 8:
            break
    verts = pts[np.sort(hull.vertices)] - com
    evals, evecs = np.linalg.eigh(inertia)
    if np.linalg.det(evecs) < 0:
        evecs[:, 2] = -evecs[:, 2]
    verts = verts @ evecs
    return verts


def _arm(osc_kp=150.0):
    """The arm, gripper, actuators and OSC configuration (bodies 1..11 after the world)."""
    rng = np.random.default_rng(1234)      # fixed robot: link masses U[0.5, 4] kg
    masses = rng.uniform(0.5, 4.0, size=7)
    bodies = []
    robot_geom = dict(contype=1, conaffinity=0, condim=3, friction=(1.0, 0.005, 0.0001))
    bodies.append(Body('base', 0, pos=(0.0, 0.0, 0.8), mass=4.0, inertia=(0.02, 0.02, 0.02),
                       ipos=(0.0, 0.0, 0.05)))
    offsets = [(0, 0, 0.333), (0, 0, 0), (0, 0, 0.316), (0.0825, 0, 0), (-0.0825, 0, 0.384),
               (0, 0, 0), (0.088, 0, 0)]
    axes = [(0, 0, 1), (0, 1, 0), (0, 0, 1), (0, 1, 0), (0, 0, 1), (0, 1, 0), (0, 0, 1)]
    spans = [0.16, 0.16, 0.16, 0.12, 0.2, 0.08, 0.08]
    parent = 1
    for k in range(7):
        length = spans[k]
        inertia = (masses[k] * (3 * 0.05 ** 2 + length ** 2) / 12,) * 2 + (masses[k] * 0.05 ** 2 / 2,)
        body = Body('link%d' % (k + 1), parent, pos=offsets[k], mass=float(masses[k]),
                    inertia=tuple(float(x) for x in inertia), ipos=(0.0, 0.0, length / 2))
        body.joints.append(Joint(HINGE, axis=axes[k], limited=True, range=(-2.9, 2.9),
                                 damping=0.1, armature=0.1))
        if k >= 5:
            body.geoms.append(Geom(CAPSULE, size=(0.045, length / 2, 0), pos=(0, 0, length / 2),
                                   **robot_geom))
        bodies.append(body)
        parent = len(bodies)
    hand = Body('hand', parent, pos=(0, 0, 0.107), mass=0.7, inertia=(0.002, 0.0015, 0.0025),
                ipos=(0, 0, 0.03))
    hand.geoms.append(Geom(BOX, size=(0.025, 0.09, 0.025), pos=(0, 0, 0.03), **robot_geom))
    hand.sites.append(Site(pos=(0, 0, 0.1034), name='grip_site'))
    bodies.append(hand)
    hand_id = len(bodies)
    for side in (1.0, -1.0):
        finger = Body('finger%s' % ('L' if side > 0 else 'R'), hand_id, pos=(0, 0, 0.0584), mass=0.1,
                      inertia=(3e-5, 3e-5, 1e-5), ipos=(0, side * 0.01, 0.03))
        finger.joints.append(Joint(SLIDE, axis=(0, side, 0), limited=True, range=(0.0, 0.04),
                                   damping=10.0, armature=0.1))
        finger.geoms.append(Geom(BOX, size=(0.008, 0.006, 0.022), pos=(0, side * 0.012, 0.032),
                                 **robot_geom))
        bodies.append(finger)
    actuators = []
    limits = [87.0, 87.0, 87.0, 87.0, 12.0, 12.0, 12.0]
    for k in range(7):
        actuators.append(Actuator(joint=k, kind='motor', ctrlrange=(-limits[k], limits[k])))
    actuators.append(Actuator(joint=7, kind='position', kp=1000.0, ctrlrange=(0.0, 0.04),
                              forcerange=(-20.0, 20.0), forcelimited=True))
    actuators.append(Actuator(joint=8, kind='position', kp=1000.0, ctrlrange=(0.0, 0.04),
                              forcerange=(-20.0, 20.0), forcelimited=True))
    # ready pose: grip site at about (0.45, 0, 1.0), gripper axis pointing down over the table
    q_ready = np.array([0.0, 0.38, 0.0, 1.89, 0.0, 0.87, 0.0])
    osc = dict(kp=np.full(6, osc_kp), kd=np.full(6, 2.0 * math.sqrt(osc_kp)), site=0,
               arm_joints=list(range(7)), actuators=list(range(9)), q0=q_ready,
               uncouple=1, gripper_speed=0.01)
    return bodies, actuators, osc, q_ready


def _world(table=True):
    world = Body('world', -1)
    static = dict(contype=0, conaffinity=1, condim=3, friction=(1.0, 0.005, 0.0001))
    world.geoms.append(Geom(PLANE, size=(0.0, 0.0, 1.0), **static))
    if table:
        world.geoms.append(Geom(BOX, size=(0.35, 0.5, 0.4), pos=(0.55, 0.0, 0.4), **static))
    return world


TABLE_TOP = 0.8
TABLE_X = (0.30, 0.80)
TABLE_Y = (-0.35, 0.35)


def _object(rng, kind, name):
    density = rng.uniform(500.0, 1500.0)
    geom_kw = dict(contype=1, conaffinity=1, condim=3, friction=(1.0, 0.005, 0.0001))
    if kind == 'box':
        half = tuple(float(x) for x in rng.uniform(0.02, 0.05, size=3))
        mass = density * 8 * half[0] * half[1] * half[2]
        body = Body(name, 0, mass=mass, inertia=box_inertia(mass, half))
        body.geoms.append(Geom(BOX, size=half, **geom_kw))
        extent = half[2]
        radius = float(np.linalg.norm(half))
    elif kind == 'capsule':
        r, h = rng.uniform(0.015, 0.04), rng.uniform(0.03, 0.08)
        mass, inertia = capsule_mass_inertia(density, r, h)
        body = Body(name, 0, mass=mass, inertia=inertia)
        body.geoms.append(Geom(CAPSULE, size=(r, h, 0.0), **geom_kw))
        extent = r
        radius = r + h
        body.quat = (math.cos(math.pi / 4), math.sin(math.pi / 4), 0.0, 0.0)  # lying on its side
    else:
        npts = int(rng.integers(16, 33)) if kind == 'hull' else 24
        verts = make_hull(rng, npts, rng.uniform(0.02, 0.05, size=3))
        mass, com, inertia, _ = hull_mass_properties(verts, density)
        body = Body(name, 0, mass=mass, inertia=tuple(float(x) for x in np.diag(inertia)))
        body.geoms.append(Geom(MESH, size=(0.0, 0.0, 0.0), vertices=verts, **geom_kw))
        extent = float(-verts[:, 2].min())
        radius = float(np.linalg.norm(verts, axis=1).max())
    body.joints.append(Joint(FREE))
    return body, extent, radius


def _place(rng, objects, layers=1):
    """Non-overlapping table placements (rejection on bounding radii) with random yaw."""
    placed = []
    qpos = []
    per_layer = math.ceil(len(objects) / layers)
    for index, (body, extent, radius) in enumerate(objects):
        layer = index // per_layer
        for _ in range(2000):
            x, y = rng.uniform(*TABLE_X), rng.uniform(*TABLE_Y)
            if all((x - px) ** 2 + (y - py) ** 2 > (radius + pr + 0.005) ** 2
                   for px, py, pr, pl in placed if pl == layer):
                break
        placed.append((x, y, radius, layer))
        z = TABLE_TOP + extent + 0.005 + layer * 0.12
        yaw = rng.uniform(0.0, 2 * math.pi)
        qy = quat_yaw(yaw)
        q = _qmul(qy, body.quat)
        qpos.extend([x, y, z, *q])
    return np.array(qpos)


def _qmul(a, b):
    aw, ax, ay, az = a
    bw, bx, by, bz = b
    return (aw * bw - ax * bx - ay * by - az * bz, aw * bx + ax * bw + ay * bz - az * by,
            aw * by - ax * bz + ay * bw + az * bx, aw * bz + ax * by - ay * bx + az * bw)


def make_scene(config='c2', nworld=None, seed=0, *, nobjects=None, substeps=25):
    """Build one of the benchmark scenes; every random draw comes from ``seed``."""
    rng = np.random.default_rng(seed)
    config = str(config).lower()
    defaults = dict(c1=2, c2=1024, c3=4096, c4=8192, c5=16384)
    if config not in defaults:
        raise ValueError('unknown scene ' + config)
    nworld = defaults[config] if nworld is None else int(nworld)
    if nworld < 1:
        raise ValueError('nworld must be positive')
    arm, actuators, osc, q_ready = _arm()
    opts = Options()
    world = _world(table=config != 'c2')
    bodies = [world] + arm
    kinds = []
    layers = 1
    if config == 'c1':
        kinds = ['box'] * 3
        opts.cone, opts.nconmax = ELLIPTIC, 64
    elif config == 'c2':
        opts.disableflags = DISABLE_CONSTRAINT | DISABLE_CONTACT
        opts.nconmax = 0
    elif config == 'c3':
        kinds = ['box', 'box', 'capsule', 'capsule', 'hull', 'hull']
        opts.cone, opts.nconmax = PYRAMIDAL, 64
    elif config == 'c4':
        mix = ['box', 'capsule', 'hull24']
        kinds = [mix[k % 3] for k in range(20)]
        layers = 2
        opts.cone, opts.nconmax = PYRAMIDAL, 256
    elif config == 'c5':
        mix = ['box', 'box', 'capsule', 'capsule', 'hull', 'hull']
        kinds = [mix[k % 6] for k in range(12)]
        opts.cone, opts.nconmax = PYRAMIDAL, 64
    if nobjects is not None:
        kinds = kinds[:nobjects]
    objects = [_object(rng, kind, 'object%d' % k) for k, kind in enumerate(kinds)]
    first_object = len(bodies)
    for body, _, _ in objects:
        bodies.append(body)
    nq = 9 + 7 * len(objects)
    nv = 9 + 6 * len(objects)
    init_qpos = np.zeros((nworld, nq))
    init_qvel = np.zeros((nworld, nv))
    for w in range(nworld):
        wrng = np.random.default_rng([seed, w])
        if config == 'c2':
            init_qpos[w, :7] = q_ready + wrng.uniform(-0.5, 0.5, size=7)
        else:
            init_qpos[w, :7] = q_ready
        if objects:
            init_qpos[w, 9:] = _place(wrng, objects, layers)
    body_active = None
    if config == 'c5':
        body_active = np.ones((nworld, len(bodies)), np.int32)
        for w in range(nworld):
            count = int(np.random.default_rng([seed, w, 5]).integers(0, len(objects) + 1))
            body_active[w, first_object + count:] = 0
            for k in range(count, len(objects)):   # parked far below the floor, never collides
                init_qpos[w, 9 + 7 * k:9 + 7 * k + 3] = (10.0 + k, 10.0 * (w % 7), -5.0)
    return Scene(name=config, bodies=bodies, actuators=actuators, options=opts, nworld=nworld,
                 substeps=substeps, osc=osc, init_qpos=init_qpos, init_qvel=init_qvel,
                 body_active=body_active, seed=seed)


def make_actions(nworld, ncontrol, seed=0, *, gripper_toggle=0):
    """Seeded OSC actions U[-1,1]^7 per world and control step, shape (ncontrol, nworld, 7)."""
    rng = np.random.default_rng([seed, 77])
    actions = rng.uniform(-1.0, 1.0, size=(ncontrol, nworld, 7))
    if gripper_toggle:
        for c in range(ncontrol):
            actions[c, :, 6] = 1.0 if (c // gripper_toggle) % 2 == 0 else -1.0
    return actions
