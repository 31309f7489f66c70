"""LIBERO intake on the CPU: the MJCF-subset compiler, the BDDL reader, the task composer and scene
files (no GPU).

Pins, independent of the code under test:

* geom mass properties against numerical integration over a fine grid (sphere, box, capsule,
  cylinder, ellipsoid) and body inertia from geoms against the parallel-axis composition of two
  boxes that form one box;
* orientations against scipy's rotations (MuJoCo's lowercase euler axes move with the frame, which
  is scipy's uppercase convention), axis-angle against the rotation vector, xyaxes / zaxis by the
  axes they map;
* default classes, childclass and partial real vectors by hand-written MJCF with known answers;
* with the reference present: every asset of the 130 tasks compiles, all 130 BDDL files parse, and
  every composed task has exactly the reference's nq, nv and njnt
  (``gpu/data/libero_task_parameters.json``), and nbody / ngeom / nsite differing from it by one
  constant per robot mount (the robot stand-in replaces robosuite's Panda);
* a composed scene saved and loaded again compiles to identical model arrays, and its objects come
  to rest on the oracle.
"""
import glob
import json
import math
from pathlib import Path

import numpy as np
import pytest

from libero_hip import bddl, libero_task, mjcf, native, scene_io, scene as S
from libero_hip.model import Model

REF = Path('/root/reference/libero/libero')
GOLDEN = Path(__file__).resolve().parent / 'golden'
needs_reference = pytest.mark.skipif(not REF.is_dir(), reason='LIBERO sources not present')


def _geom(gtype, size, **kw):
    a = dict(name='', type=gtype, size=tuple(size), pos=np.zeros(3), quat=np.array([1.0, 0, 0, 0]), group=0,
             contype=1, conaffinity=1, condim=3, priority=0, friction=(1, 0.005, 0.0001), solref=(0.02, 1),
             solimp=(0.9, 0.95, 0.001, 0.5, 2), solmix=1.0, margin=0.0, gap=0.0, density=1000.0, mass=None, mesh=None)
    a.update(kw)
    return mjcf.XGeom(**a)


def _grid_integral(inside, half_extent, n=160):
    """Volume and unit-density inertia of the set `inside` by midpoint sampling of a box grid."""
    ax = [np.linspace(-h, h, n, endpoint=False) + h / n for h in half_extent]
    x, y, z = np.meshgrid(*ax, indexing='ij')
    m = inside(x, y, z)
    dv = np.prod([2 * h / n for h in half_extent])
    vol = m.sum() * dv
    ixx = ((y * y + z * z) * m).sum() * dv
    iyy = ((x * x + z * z) * m).sum() * dv
    izz = ((x * x + y * y) * m).sum() * dv
    return vol, np.array([ixx, iyy, izz])


@pytest.mark.parametrize('gtype,size,inside,extent', [
    (S.SPHERE, (0.05,), lambda x, y, z: x * x + y * y + z * z <= 0.05 ** 2, (0.05, 0.05, 0.05)),
    (S.BOX, (0.03, 0.05, 0.02), lambda x, y, z: np.ones_like(x, bool), (0.03, 0.05, 0.02)),
    (S.CAPSULE, (0.02, 0.05), lambda x, y, z: x * x + y * y + np.maximum(np.abs(z) - 0.05, 0) ** 2 <= 0.02 ** 2,
     (0.02, 0.02, 0.07)),
    (S.CYLINDER, (0.03, 0.04), lambda x, y, z: x * x + y * y <= 0.03 ** 2, (0.03, 0.03, 0.04)),
    (S.ELLIPSOID, (0.02, 0.03, 0.05), lambda x, y, z: (x / 0.02) ** 2 + (y / 0.03) ** 2 + (z / 0.05) ** 2 <= 1,
     (0.02, 0.03, 0.05)),
])
def test_geom_mass_properties_match_integration(gtype, size, inside, extent):
    g = _geom(gtype, tuple(size) + (0.0,) * (3 - len(size)), density=700.0)
    mass, inertia = mjcf.geom_mass(g)
    vol, unit = _grid_integral(inside, extent)
    np.testing.assert_allclose(mass, 700.0 * vol, rtol=3e-3)
    np.testing.assert_allclose(inertia, 700.0 * unit, rtol=6e-3)
    # an explicit mass scales the same distribution
    g.mass = 2.5
    m2, i2 = mjcf.geom_mass(g)
    assert m2 == 2.5
    np.testing.assert_allclose(i2, inertia * 2.5 / mass, rtol=1e-12)


def test_body_inertia_from_two_boxes_is_one_box():
    q = mjcf.axis_quat((0.3, -0.5, 0.8), 0.7)
    R = mjcf.quat2mat(q)
    centre = np.array([0.1, -0.2, 0.05])
    halves = (0.02, 0.03, 0.05)
    parts = [_geom(S.BOX, halves, pos=centre + R @ np.array([s * 0.02, 0, 0]), quat=q) for s in (-1, 1)]
    mass, com, principal, frame = mjcf.inertia_from_geoms(parts)
    whole = _geom(S.BOX, (0.04, 0.03, 0.05))
    m1, i1 = mjcf.geom_mass(whole)
    np.testing.assert_allclose(mass, m1, rtol=1e-12)
    np.testing.assert_allclose(com, centre, atol=1e-15)
    np.testing.assert_allclose(sorted(principal), sorted(i1), rtol=1e-10)
    # the principal frame maps the body's axes to the box's (up to axis order and sign)
    Rf = mjcf.quat2mat(frame)
    full = Rf @ np.diag(principal) @ Rf.T
    np.testing.assert_allclose(full, R @ np.diag(i1) @ R.T, atol=1e-12 * i1.max())


@pytest.mark.parametrize('seq', ['xyz', 'XYZ', 'zyx', 'ZYX', 'yzx'])
def test_euler_sequences_match_scipy(seq):
    from scipy.spatial.transform import Rotation
    angles = (0.4, -1.1, 2.3)
    comp = mjcf.Compiler(angle='radian', eulerseq=seq)
    q = mjcf.orientation({'euler': ' '.join(map(str, angles))}, comp)
    # MuJoCo: lowercase axes rotate with the frame (scipy: uppercase), uppercase are fixed
    ref = Rotation.from_euler(seq.swapcase(), angles).as_matrix()
    np.testing.assert_allclose(mjcf.quat2mat(q), ref, atol=1e-12)
    comp_deg = mjcf.Compiler(angle='degree', eulerseq=seq)
    qd = mjcf.orientation({'euler': ' '.join(str(math.degrees(a)) for a in angles)}, comp_deg)
    np.testing.assert_allclose(mjcf.quat2mat(qd), ref, atol=1e-12)


def test_axisangle_xyaxes_zaxis():
    from scipy.spatial.transform import Rotation
    comp = mjcf.Compiler(angle='degree')
    q = mjcf.orientation({'axisangle': '1 2 2 60'}, comp)
    ref = Rotation.from_rotvec(np.array([1, 2, 2]) / 3 * math.radians(60)).as_matrix()
    np.testing.assert_allclose(mjcf.quat2mat(q), ref, atol=1e-12)
    R = mjcf.quat2mat(mjcf.orientation({'xyaxes': '0 1 0 -1 0 0'}, comp))
    np.testing.assert_allclose(R @ [1, 0, 0], [0, 1, 0], atol=1e-12)
    np.testing.assert_allclose(R @ [0, 1, 0], [-1, 0, 0], atol=1e-12)
    z = np.array([1.0, 1.0, 1.0]) / math.sqrt(3)
    R = mjcf.quat2mat(mjcf.orientation({'zaxis': '1 1 1'}, comp))
    np.testing.assert_allclose(R @ [0, 0, 1], z, atol=1e-12)
    np.testing.assert_allclose(mjcf.quat2mat(mjcf.mat2quat(R)), R, atol=1e-12)


XML = """
<mujoco model="t">
  <compiler angle="radian" inertiagrouprange="0 0"/>
  <default>
    <geom density="500" friction="0.7"/>
    <default class="soft">
      <geom solref="0.05 0.8" solimp="0.8 0.9 0.002"/>
      <default class="softer"><geom solimp="0.5"/></default>
    </default>
    <joint damping="0.3"/>
  </default>
  <worldbody>
    <geom type="plane" size="1 1 0.1"/>
    <body name="a" pos="0 0 1" childclass="soft">
      <joint type="hinge" axis="0 1 0" range="-1 1"/>
      <geom type="box" size="0.1 0.1 0.1"/>
      <geom type="box" size="0.1 0.1 0.1" pos="0 0 0.5" group="1" contype="0" conaffinity="0"/>
      <geom type="mesh" mesh="vis" group="1" contype="0" conaffinity="0"/>
      <body name="b" pos="0.2 0 0">
        <joint type="slide" axis="1 0 0"/>
        <inertial pos="0 0 0.1" mass="2" fullinertia="3 2 1 0 0 0"/>
        <geom class="softer" type="sphere" size="0.05"/>
        <geom class="main" type="sphere" size="0.05" pos="0.1 0 0"/>
        <site name="s" pos="0 0 0.2" euler="0 0 1.5707963267948966"/>
      </body>
    </body>
  </worldbody>
</mujoco>
"""


def test_defaults_classes_and_compile_rules():
    comp_model = mjcf.load(XML)
    comp = comp_model.compiler
    assert comp.angle == 'radian' and comp.inertiagrouprange == (0, 0)
    bodies = mjcf.compile_bodies(comp_model.world, comp)
    world, a, b = bodies
    assert [bd.parent for bd in bodies] == [-1, 0, 1]
    # body a: only the group-0 box carries mass (visual box and visual mesh excluded), density 500
    np.testing.assert_allclose(a.mass, 500 * 0.2 ** 3)
    assert len(a.geoms) == 1                               # visual geoms dropped from the model
    g = a.geoms[0]
    assert g.friction == (0.7, 0.005, 0.0001)              # main class, prefix filled from MuJoCo's
    assert g.solref == (0.05, 0.8) and g.solimp == (0.8, 0.9, 0.002, 0.5, 2.0)   # childclass soft
    ja = a.joints[0]
    assert ja.limited and ja.range == (-1.0, 1.0) and ja.damping == 0.3
    # body b: <inertial> (auto) with fullinertia diagonalised; no range -> not limited (autolimits)
    assert b.mass == 2.0 and sorted(b.inertia) == [1.0, 2.0, 3.0] and b.ipos == (0.0, 0.0, 0.1)
    assert not b.joints[0].limited
    soft, plain = b.geoms
    assert soft.solimp == (0.5, 0.9, 0.002, 0.5, 2.0) and soft.solref == (0.05, 0.8)   # softer < soft
    assert plain.solref == (0.02, 1.0) and plain.friction[0] == 0.7                 # class main
    np.testing.assert_allclose(mjcf.quat2mat(b.sites[0].quat) @ [1, 0, 0], [0, 1, 0], atol=1e-12)
    # inertiafromgeom true overrides <inertial>
    comp2 = mjcf.Compiler(angle='radian', inertiagrouprange=(0, 0), inertiafromgeom='true')
    b2 = mjcf.compile_bodies(mjcf.load(XML, compiler=comp2).world, comp2)[2]
    np.testing.assert_allclose(b2.mass, 2 * 500 * 4 / 3 * math.pi * 0.05 ** 3)
    # the visual mesh carries mass when its group is in the inertia range: its data is absent
    comp3 = mjcf.Compiler(angle='radian', inertiagrouprange=(0, 1))
    with pytest.raises(mjcf.MjcfError, match='mesh'):
        mjcf.compile_bodies(mjcf.load(XML, compiler=comp3).world, comp3)
    with pytest.raises(mjcf.MjcfError, match='mesh'):
        mjcf.compile_bodies(mjcf.load(XML.replace('contype="0" conaffinity="0"/>\n      <body',
                                                  '/>\n      <body'), compiler=comp).world, comp)


def test_sexpr_and_bddl_text():
    text = """(define (problem LIBERO_Tabletop_Manipulation) ; comment
      (:domain robosuite)
      (:language put the bowl on the plate)
      (:regions (plate_region (:target main_table) (:ranges ((0.1 0.2 0.3 0.4))) (:yaw_rotation ((0.5 0.6)))))
      (:fixtures main_table - table cab_1 - wooden_cabinet)
      (:objects bowl_1 bowl_2 - akita_black_bowl plate_1 - plate)
      (:obj_of_interest bowl_1)
      (:init (On bowl_1 main_table_plate_region) (Open cab_1_top_region))
      (:goal (And (On bowl_1 plate_1))))"""
    p = bddl.parse(text)
    assert p.name == 'LIBERO_Tabletop_Manipulation' and p.language == 'put the bowl on the plate'
    r = p.regions['main_table_plate_region']
    assert r.target == 'main_table' and r.ranges == [(0.1, 0.2, 0.3, 0.4)] and r.yaw_rotation == (0.5, 0.6)
    assert p.fixtures == {'table': ['main_table'], 'wooden_cabinet': ['cab_1']}
    assert p.objects == {'akita_black_bowl': ['bowl_1', 'bowl_2'], 'plate': ['plate_1']}
    assert p.init == [('on', 'bowl_1', 'main_table_plate_region'), ('open', 'cab_1_top_region')]
    assert p.goal == ['And', ['On', 'bowl_1', 'plate_1']]
    assert p.category('bowl_2') == 'akita_black_bowl' and p.is_fixture('cab_1')
    with pytest.raises(bddl.BddlError):
        bddl.parse_sexpr('(a (b)')


@needs_reference
def test_all_task_assets_compile_and_bddl_parse():
    comp = libero_task.robosuite_compiler()
    files = sorted(glob.glob(str(REF / 'bddl_files' / '*' / '*.bddl')))
    assert len(files) == 130
    cats = set()
    for f in files:
        p = bddl.parse(f)
        cats |= {c for c in list(p.fixtures) + list(p.objects) if c not in libero_task.PROBLEMS_WORKSPACES}
    for c in sorted(cats):
        path, folder = libero_task.asset_path(REF / 'assets', c)
        mjcf.compile_bodies(mjcf.load(path, compiler=comp).world, comp)
    for spec in libero_task.PROBLEMS.values():
        mjcf.compile_bodies(mjcf.load(REF / 'assets' / spec['arena'], compiler=comp).world, comp)


@needs_reference
def test_composed_tasks_match_the_reference_dimensions():
    catalog = json.loads((REF / 'gpu' / 'data' / 'libero_task_parameters.json').read_text())
    dims = {t['key']: t['dimensions'] for t in catalog['tasks']}
    offsets = {}
    for f in sorted(glob.glob(str(REF / 'bddl_files' / '*' / '*.bddl'))):
        key = '/'.join(Path(f).parts[-2:])
        task = libero_task.compose(f, REF / 'assets', nworld=1, seed=0)
        m = Model(task.scene)
        d = dims[key]
        assert (m.nq, m.nv, m.njnt) == (d['nq'], d['nv'], d['njnt']), key
        assert m.nu == d['nu'] and m.nsensor == d['nsensor']
        mount = 'ground' if task.problem.name.lower() in ('libero_living_room_tabletop_manipulation',
                                                          'libero_floor_manipulation') else 'mounted'
        diff = tuple(d[k] - task.counts[k] for k in ('nbody', 'ngeom', 'nsite'))
        offsets.setdefault(mount, set()).add(diff)
    # the robot's share is the same in every task of a mount
    assert all(len(v) == 1 for v in offsets.values()), offsets


@needs_reference
def test_saved_scene_round_trip(tmp_path):
    f = REF / 'bddl_files' / 'libero_spatial' / \
        'pick_up_the_black_bowl_between_the_plate_and_the_ramekin_and_place_it_on_the_plate.bddl'
    task = libero_task.compose(f, REF / 'assets', nworld=16, seed=0)
    scene_io.save(task.scene, tmp_path / 's.json')
    a, b = Model(task.scene), Model(scene_io.load(tmp_path / 's.json'))
    for k, v in a.arrays.items():
        np.testing.assert_array_equal(v, b.arrays[k], err_msg=k)
    # the committed fixture is this composition
    c = Model(scene_io.load(GOLDEN / 'libero_spatial_bowl_plate.json'))
    for k, v in a.arrays.items():
        np.testing.assert_array_equal(v, c.arrays[k], err_msg=k)
    np.testing.assert_array_equal(task.scene.init_qpos, scene_io.load(GOLDEN / 'libero_spatial_bowl_plate.json').init_qpos)


@pytest.mark.parametrize('name', ['libero_spatial_bowl_plate', 'libero_living_room_basket', 'libero_object_soup_basket',
                                  'libero_goal_wine_rack', 'libero_10_mugs_plates'])
def test_saved_scene_objects_come_to_rest(name):
    from helpers import make_oracle
    sc = scene_io.load(GOLDEN / (name + '.json'))
    sc.nworld = 2
    sc.init_qpos, sc.init_qvel = sc.init_qpos[:2], sc.init_qvel[:2]
    m = Model(sc)
    om, od = make_oracle(m, 2)
    od['qpos'][:] = sc.init_qpos
    od.forward(None, native.FLAG_BOOTSTRAP | native.FLAG_NO_CONTROL)
    nobj = sum(1 for b in sc.bodies if b.joints and b.joints[0].type == S.FREE)
    for _ in range(40):                                    # 2 s, the arm holding its pose
        od['osc_action'][:] = 0
        od.control_step(25, native.FLAG_POLICY_FIRST)
    assert not od['overflow'].any()
    v = od['qvel'][:, -6 * nobj:].reshape(2, nobj, 6)
    assert np.abs(v[..., :3]).max() < 0.05                 # linear speeds (m/s)
    z = od['qpos'][:, -7 * nobj:].reshape(2, nobj, 7)[..., 2]
    assert (z > 0.0).all()
