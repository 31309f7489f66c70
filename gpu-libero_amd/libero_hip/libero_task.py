"""LIBERO task scenes from BDDL files and LIBERO's asset MJCF.

The reference builds each task with robosuite and CPU MuJoCo (``gpu/host/backends/cuda_fp32/scene.py:88-143``
``build_scene`` -> ``libero.gpu.model.build_task_model``): the problem class picks the arena and the
workspace (``libero/libero/envs/problems/*.py``), the BDDL file names the fixtures and objects, and
robosuite merges the arena, the robot and every object into one model compiled with robosuite's base
compiler settings (angles in radians; only group-0 geoms carry mass).  This module composes the same
content into a :class:`~libero_hip.scene.Scene` with :mod:`libero_hip.mjcf`:

* the arena XML of the problem (``libero/libero/envs/arenas``: tabletop and kitchen tables resized to
  the problem's table size, offset and friction as ``TableArena.configure_location`` does; study,
  living-room and floor arenas as written) as static bodies, plus one site per workspace region;
* the robot stand-in: robosuite's Panda model is not part of the reference, so the backend's
  7-revolute arm with its 2-slide gripper (the same 9 joints, 7 + 2 actuators and OSC layout) stands
  at the robot base position the problem gives (``robots/mounted_panda.py`` ``base_xpos_offset``);
* fixtures (``joints=None``: welded, their articulation joints kept) at a seeded placement in their
  region (yaw from the region, ``z_offset`` of the problem) and objects with a free joint (damping
  0.0005) placed per world in their regions with the object class's rotation (``regions/
  base_region_sampler.py`` ``MultiRegionRandomSampler``); objects on fixture regions or on other
  objects are placed at the target site or on top of the target object;
* options of LIBERO's scenes (``gpu/data/libero_task_parameters.json``): timestep 0.002, elliptic
  cones, impratio 20, medium density 1.2 and viscosity 2e-5, 100 Newton iterations with the FP32
  tolerance floor 1e-6, capacities as ``capacity_budget`` (``scene.py:71-86``) sizes them.

The official initial states (``init_files/*.pruned_init``) are not in the reference, so initial poses
are sampled; the placement rules above are the ones LIBERO samples new episodes with.
"""
from __future__ import annotations

from dataclasses import dataclass, field
import math
from pathlib import Path

import numpy as np

from . import bddl, mjcf, scene as S

PI = math.pi

# problem -> arena file, workspace fixture, table size / offset / friction, robot base rule, the
# fixtures' z offset (libero/libero/envs/problems/*.py, bddl_base_domain.py:308-392)
PROBLEMS = {
    'libero_tabletop_manipulation': dict(
        arena='scenes/libero_tabletop_base_style.xml', workspace='main_table', resize='table',
        size=(1.0, 1.2, 0.05), offset=(0.0, 0.0, 0.90), friction=(0.6, 0.005, 0.0001),
        robot=lambda size, off: (-0.16 - size[0] / 2, 0.0, off[2])),
    'libero_kitchen_tabletop_manipulation': dict(
        arena='scenes/libero_kitchen_tabletop_base_style.xml', workspace='kitchen_table', resize='table',
        size=(1.0, 1.2, 0.05), offset=(0.0, 0.0, 0.90), friction=(1.0, 0.005, 0.0001),
        robot=lambda size, off: (-0.16 - size[0] / 2, 0.0, off[2])),
    'libero_living_room_tabletop_manipulation': dict(
        arena='scenes/libero_living_room_tabletop_base_style.xml', workspace='living_room_table', resize=None,
        size=(0.70, 1.6, 0.024), offset=(0.0, 0.0, 0.41),
        robot=lambda size, off: (-0.16 - size[0] / 2, 0.0, 0.42)),
    'libero_study_tabletop_manipulation': dict(
        arena='scenes/libero_study_base_style.xml', workspace='study_table', resize=None,
        size=(1.0, 1.2, 0.05), offset=(-0.2, 0.0, 0.867),
        robot=lambda size, off: (-0.25 - size[0] / 2, 0.0, off[2])),
    'libero_floor_manipulation': dict(
        arena='scenes/libero_floor_base_style.xml', workspace='floor', resize=None,
        size=None, offset=(0.0, 0.0, -0.035), z_offset=-0.025,
        robot=lambda size, off: (-0.6, 0.0, 0.0)),
}

# object class placement rotations (libero/libero/envs/objects/*.py: rotation, rotation_axis);
# a dict composes its axes in order, each about the world axis
_X90 = ('x', (PI / 2, PI / 2))
ROTATIONS = {
    # stable_scanned_objects (GoogleScannedObject)
    'akita_black_bowl': _X90, 'white_bowl': _X90, 'plate': _X90, 'basket': _X90, 'red_bowl': _X90,
    'chefmate_8_frypan': _X90, 'glazed_rim_porcelain_ramekin': _X90, 'simple_rack': ('x', (0.0, 0.0)),
    # stable_hope_objects (HopeBaseObject)
    'alphabet_soup': ('z', (PI / 2, PI / 2)), 'tomato_sauce': ('z', (PI / 2, PI / 2)),
    'bbq_sauce': _X90, 'cookies': _X90, 'butter': ('x', (0.0, 0.0)), 'chocolate_pudding': ('x', (0.0, 0.0)),
    'cream_cheese': ('x', (0.0, 0.0)), 'popcorn': ('x', (0.0, 0.0)),
    'ketchup': {'x': (PI / 2, PI / 2), 'z': (PI / 2, PI / 2)},
    'macaroni_and_cheese': {'x': (PI / 2, PI / 2), 'z': (PI / 2, PI / 2)},
    'milk': {'x': (PI / 2, PI / 2), 'z': (PI / 2, PI / 2)},
    'orange_juice': {'x': (PI / 2, PI / 2), 'z': (PI / 2, PI / 2)},
    'salad_dressing': {'x': (PI / 2, PI / 2), 'z': (PI / 2, PI / 2)},
    'new_salad_dressing': {'x': (PI / 2, PI / 2), 'z': (PI / 2, PI / 2)},
    # turbosquid_objects
    'black_book': ('x', (-PI / 2, -PI / 4)), 'yellow_book': ('x', (-PI / 2, -PI / 4)),
    'red_coffee_mug': ('x', (-PI / 2, -PI / 2)), 'porcelain_mug': ('x', (-PI / 2, -PI / 2)),
    'white_yellow_mug': ('x', (-PI / 2, -PI / 2)), 'white_storage_box': ('y', (0.0, 0.0)),
    # articulated_objects
    'flat_stove': ('y', (0.0, 0.0)),
}
DEFAULT_ROTATION = {'turbosquid_objects': ('x', (0.0, 0.0)), 'articulated_objects': ('x', (PI / 4, PI / 2)),
                    'stable_scanned_objects': _X90, 'stable_hope_objects': _X90}

# articulation ranges of the initial relations (objects/articulated_objects.py)
ARTICULATION = {
    'microwave': dict(open=(-2.094, -1.3), close=(-0.005, 0.0)),
    'short_cabinet': dict(open=(0.10, 0.16), close=(-0.005, 0.0)),
    'short_fridge': dict(open=(2.0, 2.7), close=(-0.005, 0.0)),
    'wooden_cabinet': dict(open=(-0.16, -0.14), close=(0.0, 0.005)),
    'white_cabinet': dict(open=(-0.16, -0.14), close=(0.0, 0.005)),
    'flat_stove': dict(turnon=(0.5, 2.1), turnoff=(-0.005, 0.0)),
}

OBJECT_DAMPING = 0.0005       # free joints of movable objects (objects/*.py joints=[dict(type="free", ...)])
REGION_Z_OFFSET = 0.01        # TableRegionSampler z_offset (regions/workspace_region_sampler.py)


def robosuite_compiler():
    """The compiler a composed LIBERO scene is built with (robosuite's merged model)."""
    return mjcf.Compiler(angle='radian', inertiagrouprange=(0, 0))


def asset_path(root, category):
    """The asset file of an object or fixture category (objects/*.py asset folders)."""
    root = Path(root)
    for folder in ('stable_scanned_objects', 'stable_hope_objects', 'turbosquid_objects'):
        p = root / folder / category / (category + '.xml')
        if p.is_file():
            return p, folder
    p = root / 'articulated_objects' / (category + '.xml')
    if p.is_file():
        return p, 'articulated_objects'
    raise FileNotFoundError('no asset for category %r under %s' % (category, root))


@dataclass
class Asset:
    """One object or fixture instance: its compiled subtree and placement offsets."""
    name: str
    category: str
    fixture: bool
    body: mjcf.XBody                 # the 'object' body (renamed to the instance)
    bottom: np.ndarray
    top: np.ndarray
    radius: float
    rotation: object

    def site(self, name):
        """Pose (pos, quat) of a named site in the object's frame, with the joints of its body."""
        def walk(xb, pos, quat):
            R = mjcf.quat2mat(quat)
            for s in xb.sites:
                if s.name == name:
                    return pos + R @ np.asarray(s.pos), mjcf.qmul(quat, s.quat), xb
            for ch in xb.children:
                hit = walk(ch, pos + R @ ch.pos, mjcf.qmul(quat, ch.quat))
                if hit:
                    return hit
            return None
        return walk(self.body, np.zeros(3), np.array([1.0, 0.0, 0.0, 0.0]))


def load_asset(root, instance, category, fixture, compiler):
    path, folder = asset_path(root, category)
    model = mjcf.load(path, compiler=compiler)
    outer = model.world.children
    if len(outer) != 1:
        raise mjcf.MjcfError('%s: expected one top-level body' % path)
    outer = outer[0]
    obj = next((b for b in outer.children if b.name == 'object'), None)
    if obj is None:
        raise mjcf.MjcfError("%s: no body named 'object'" % path)
    sites = {s.name: np.asarray(s.pos, float) for s in outer.sites}
    bottom = sites.get('bottom_site', np.zeros(3))
    top = sites.get('top_site', np.zeros(3))
    radius = float(np.linalg.norm(sites.get('horizontal_radius_site', np.zeros(3))[:2]))
    obj.name = instance
    rot = ROTATIONS.get(category, DEFAULT_ROTATION[folder])
    return Asset(instance, category, fixture, obj, bottom, top, radius, rot)


def sample_quat(rng, rotation, axis_default='z'):
    """Orientation of a placement: an angle uniform in an interval about one axis, or a dict of
    axes composed in order (each later rotation applied about the world axis)."""
    def about(axis, lo_hi):
        lo, hi = min(lo_hi), max(lo_hi)
        a = rng.uniform(lo, hi) if hi > lo else lo
        return mjcf.axis_quat(np.eye(3)['xyz'.index(axis)], a)
    if isinstance(rotation, dict):
        q = np.array([1.0, 0.0, 0.0, 0.0])
        for axis, lo_hi in rotation.items():
            q = mjcf.qmul(about(axis, lo_hi), q)
        return q
    axis, lo_hi = rotation if isinstance(rotation, tuple) and isinstance(rotation[0], str) else (axis_default, rotation)
    return about(axis, lo_hi)


@dataclass
class Task:
    """A composed task: the scene plus what the composition decided."""
    scene: S.Scene
    problem: bddl.Problem
    counts: dict                     # MuJoCo-style counts of the non-robot part (visual geoms included)
    objects: list                    # movable object instance names, in body order
    fixtures: list
    fixture_pose: dict = field(default_factory=dict)


def _arena(root, spec, problem, compiler):
    model = mjcf.load(Path(root) / spec['arena'], compiler=compiler)
    world = model.world
    ws = problem_workspace_regions(problem, spec['workspace'])
    if spec['resize'] == 'table':
        half = np.asarray(spec['size']) / 2
        table = next(b for b in world.children if b.name == 'table')
        table.pos = np.array([0.0, 0.0, -half[2]]) + np.asarray(spec['offset'])
        for g in table.geoms:
            if g.name in ('table_collision', 'table_visual'):
                g.size = tuple(half)
            if g.name == 'table_collision':
                g.friction = tuple(spec['friction'])
        for s in table.sites:
            if s.name == 'table_top':
                s.pos = (0.0, 0.0, half[2])
        anchor = table
    else:
        anchor = world
    # one site per workspace region at its centre (problems/*.py _load_sites_in_arena)
    for key, region in ws.items():
        x0, y0, x1, y1 = region.ranges[0]
        base = np.asarray(spec['offset']) - (anchor.pos if anchor is not world else 0.0)
        anchor.sites.append(S.Site(pos=(float(base[0] + (x0 + x1) / 2), float(base[1] + (y0 + y1) / 2),
                                        float(base[2])), name=key))
    return world


def problem_workspace_regions(problem, workspace):
    return {k: r for k, r in problem.regions.items() if r.target == workspace and r.ranges}


def capacity(nv, cone):
    """capacity_budget (gpu/host/backends/cuda_fp32/scene.py:71-86) for condim-3 contacts."""
    power2 = lambda v: 1 << (int(v) - 1).bit_length()
    nconmax = max(256, power2(4 * nv))
    rows = 3 if cone == S.ELLIPTIC else 4
    return nconmax, max(512, power2(rows * nconmax + 2 * nv))


def compose(bddl_file, assets_root, *, nworld=1, seed=0, substeps=25, nconmax=None):
    """Scene of a LIBERO task: arena, robot stand-in, fixtures and objects (see the module notes)."""
    problem = bddl.parse(bddl_file)
    key = problem.name.lower()
    if key not in PROBLEMS:
        raise ValueError('unknown LIBERO problem %s' % problem.name)
    spec = PROBLEMS[key]
    comp = robosuite_compiler()
    rng = np.random.default_rng([seed, 101])
    world = _arena(assets_root, spec, problem, comp)
    workspace = spec['workspace']
    z_fixture = spec.get('z_offset', REGION_Z_OFFSET - (spec['size'][2] if spec['size'] else 0.0))
    offset = np.asarray(spec['offset'])

    fixtures, objects = [], []
    for cat, names in problem.fixtures.items():
        if cat in PROBLEMS_WORKSPACES:
            continue
        for n in names:
            fixtures.append(load_asset(assets_root, n, cat, True, comp))
    for cat, names in problem.objects.items():
        for n in names:
            objects.append(load_asset(assets_root, n, cat, False, comp))
    by_name = {a.name: a for a in fixtures + objects}
    init = {rel[1]: rel for rel in problem.init if rel[0] in ('on', 'in')}

    # fixtures: one seeded placement, welded into the world
    poses = {}
    for a in fixtures:
        rel = init.get(a.name)
        if rel is None or rel[2] not in problem.regions:
            raise ValueError('fixture %s has no workspace region' % a.name)
        region = problem.regions[rel[2]]
        x0, y0, x1, y1 = region.ranges[rng.integers(len(region.ranges))]
        pos = np.array([rng.uniform(x0, x1), rng.uniform(y0, y1), z_fixture]) + offset
        pos[2] -= a.bottom[2]
        quat = sample_quat(rng, ('z', region.yaw_rotation))
        poses[a.name] = (pos, quat)
        a.body.pos, a.body.quat = pos, quat
        world.children.append(a.body)

    # the robot stand-in
    arm, actuators, osc, q_ready = S._arm()
    base = np.asarray(spec['robot'](spec['size'], offset))
    arm[0].pos = tuple(base)

    # objects: free bodies after the fixtures
    for a in objects:
        a.body.joints = [S.Joint(S.FREE, damping=OBJECT_DAMPING)]
        a.body.joint_names = [a.name + '_joint0']
        a.body.pos, a.body.quat = np.zeros(3), np.array([1.0, 0.0, 0.0, 0.0])
        world.children.append(a.body)

    bodies = mjcf.compile_bodies(world, comp)
    # the arm goes right after the world's static subtrees, before fixtures' and objects' own bodies:
    # bodies are kept in DFS preorder by appending it as the world's next child subtree
    arm_first = len(bodies)
    for b in arm:
        b.parent = 0 if b.parent == 0 else b.parent + arm_first - 1
    bodies = bodies + arm
    # reorder so that the arm's dofs come first (the controller's joints 0..8)
    bodies = _arm_first(bodies, arm_first, len(arm))

    nq_obj = 7 * len(objects)
    fixture_joints = [(a, j) for a in fixtures for j in _joints(a.body)]
    nfj = sum(1 for _ in fixture_joints)
    nq = 9 + nfj + nq_obj
    init_qpos = np.zeros((nworld, nq))
    init_qpos[:, :7] = q_ready
    init_qpos[:, 7:9] = 0.0
    # fixture articulation from the initial relations (open / close / turnon / turnoff)
    art = {rel[1]: rel[0] for rel in problem.init if rel[0] in ('open', 'close', 'turnon', 'turnoff')}
    for k, (a, (xb, jname)) in enumerate(fixture_joints):
        qv = 0.0
        for target, state in art.items():
            hit = _region_joint(a, target)
            if hit is not None and hit == jname and a.category in ARTICULATION:
                lo, hi = ARTICULATION[a.category][state]
                qv = 0.5 * (lo + hi)
        init_qpos[:, 9 + k] = qv
    order = _placement_order(objects, init, problem)
    for w in range(nworld):
        wrng = np.random.default_rng([seed, w, 7])
        placed = {}
        for i in order:
            a = objects[i]
            pos, quat = _place_object(a, init.get(a.name), problem, by_name, poses, placed, offset, wrng)
            placed[a.name] = (pos, quat)
            init_qpos[w, 9 + nfj + 7 * i:9 + nfj + 7 * i + 7] = [*pos, *quat]

    opts = S.Options(timestep=0.002, cone=S.ELLIPTIC, impratio=20.0, iterations=100, tolerance=1e-6,
                     density=1.2, viscosity=2e-5)
    nv = 9 + nfj + 6 * len(objects)
    cap, rows = capacity(nv, opts.cone)
    opts.nconmax = int(nconmax) if nconmax is not None else cap
    opts.njmax = 0 if nconmax is not None else rows
    # the controller's site and the robot's wrist force / torque sensors (nsensor 2 in LIBERO's scenes)
    names = [st.name for b in bodies for st in b.sites]
    osc['site'] = names.index('grip_site')
    sensors = [S.Sensor('force', osc['site']), S.Sensor('torque', osc['site'])]
    sc = S.Scene(name=key, bodies=bodies, actuators=actuators, options=opts, nworld=nworld, substeps=substeps,
                 osc=osc, init_qpos=init_qpos, init_qvel=np.zeros((nworld, nv)), seed=seed, sensors=sensors)
    counts = _counts(world, problem, spec)
    return Task(sc, problem, counts, [a.name for a in objects], [a.name for a in fixtures], poses)


PROBLEMS_WORKSPACES = {'table', 'kitchen_table', 'living_room_table', 'study_table', 'floor'}


def _joints(xb):
    for j, name in zip(xb.joints, xb.joint_names):
        yield xb, name
    for ch in xb.children:
        yield from _joints(ch)


def _region_joint(asset, target):
    """The joint name of the body that holds the region site `target` (an instance-prefixed site)."""
    prefix = asset.name + '_'
    if not target.startswith(prefix):
        return None
    hit = asset.site(target[len(prefix):])
    if hit is None or not hit[2].joint_names:
        return None
    return hit[2].joint_names[0]


def _placement_order(objects, init, problem):
    """Object indices with every object after the object it is placed on or in."""
    names = {a.name: i for i, a in enumerate(objects)}

    def host(a):
        rel = init.get(a.name)
        if rel is None:
            return None
        t = rel[2]
        t = problem.regions[t].target if t in problem.regions else t
        return names.get(t)
    order, done = [], set()
    while len(order) < len(objects):
        progress = False
        for i, a in enumerate(objects):
            h = host(a)
            if i not in done and (h is None or h in done):
                order.append(i)
                done.add(i)
                progress = True
        if not progress:
            raise ValueError('circular placement relations')
    return order


def _place_object(a, rel, problem, by_name, fixture_poses, placed, offset, rng):
    """Initial pose of a movable object from its On / In relation."""
    quat = sample_quat(rng, a.rotation, 'x')
    if rel is None:
        raise ValueError('object %s has no initial relation' % a.name)
    target = rel[2]
    if target in problem.regions and problem.regions[target].target in PROBLEMS_WORKSPACES | _workspace_names(problem):
        region = problem.regions[target]
        for _ in range(5000):
            x0, y0, x1, y1 = region.ranges[rng.integers(len(region.ranges))]
            x, y = rng.uniform(x0, x1) + offset[0], rng.uniform(y0, y1) + offset[1]
            ok = all(math.hypot(x - p[0][0], y - p[0][1]) > a.radius + by_name[n].radius
                     for n, p in placed.items())
            if ok:
                break
        return np.array([x, y, REGION_Z_OFFSET + offset[2] - a.bottom[2]]), quat
    if target in problem.regions:
        # a region of a fixture or object: the site of that name on the target, sampled over its extent
        region = problem.regions[target]
        host = by_name[region.target]
        hit = host.site(region.name)
        pose = fixture_poses.get(host.name, placed.get(host.name))
        if hit is None or pose is None:
            raise ValueError('no site %s on %s' % (region.name, host.name))
        hpos, hquat = pose
        spos = hpos + mjcf.quat2mat(hquat) @ hit[0]
        return np.array([spos[0], spos[1], spos[2] + REGION_Z_OFFSET - a.bottom[2]]), quat
    if target in placed:
        # on another object: on top of it
        tpos = placed[target][0]
        t = by_name[target]
        return np.array([tpos[0], tpos[1], tpos[2] + t.top[2] - a.bottom[2] + REGION_Z_OFFSET]), quat
    raise ValueError('cannot place %s on %s' % (a.name, target))


def _workspace_names(problem):
    return {n for cat, names in problem.fixtures.items() if cat in PROBLEMS_WORKSPACES for n in names}


def _arm_first(bodies, arm_first, narm):
    """Move the arm's subtree to directly after the world (body 1), keeping DFS preorder."""
    order = [0] + list(range(arm_first, arm_first + narm)) + list(range(1, arm_first))
    new_index = {old: new for new, old in enumerate(order)}
    out = []
    for old in order:
        b = bodies[old]
        b.parent = -1 if old == 0 else new_index[b.parent]
        out.append(b)
    return out


def _counts(world, problem, spec):
    """MuJoCo counts of the composed non-robot part (every geom and site; robosuite adds one site per
    object and fixture)."""
    nbody, njnt, ngeom, nsite, nq, nv = mjcf.counts(world, include_self=False)
    ninst = sum(len(v) for c, v in problem.fixtures.items() if c not in PROBLEMS_WORKSPACES) + \
        sum(len(v) for v in problem.objects.values())
    return dict(nbody=nbody, njnt=njnt, ngeom=ngeom, nsite=nsite + ninst, nq=nq, nv=nv)
