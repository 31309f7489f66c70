"""MJCF-subset compiler: LIBERO asset XML -> :class:`~libero_hip.scene.Body` trees.

The reference compiles LIBERO's scenes with CPU MuJoCo (``gpu/host/backends/cuda_fp32/scene.py:88-143``,
``build_task_model``) and preprocesses the compiled model (``model.py:27-191``).  MuJoCo is not part
of this backend, so the subset of MJCF that LIBERO's asset files use is compiled here, with MuJoCo's
documented compile semantics:

* ``<compiler>``: ``angle`` (degree or radian), ``eulerseq``, ``inertiafromgeom`` (auto / true /
  false), ``inertiagrouprange``, ``autolimits``, ``boundmass`` / ``boundinertia``;
* ``<default>`` classes, nested (a class inherits its parent's values), selected by ``class`` on the
  element or ``childclass`` on an enclosing body, MuJoCo's built-in values underneath;
* ``<body>`` with ``pos`` and an orientation (``quat``, ``axisangle``, ``euler``, ``xyaxes``,
  ``zaxis``), ``<inertial>`` (``diaginertia`` or ``fullinertia``), ``<joint>`` (free, ball, slide,
  hinge; ``limited`` true / false / auto), ``<freejoint>``, ``<geom>`` and ``<site>``;
* geom mass from ``mass`` or ``density`` times the volume of the primitive; body inertia from the
  geoms in the inertia group range (parallel-axis sums, then principal axes) when ``inertiafromgeom``
  asks for it.

Mesh data is not shipped with LIBERO's asset XMLs in the reference (the ``.msh`` files are absent), so
a mesh geom is accepted only where it neither collides nor carries mass; a collision mesh raises.
Cameras, lights, materials and textures are ignored.
"""
from __future__ import annotations

import copy
import math
from dataclasses import dataclass, field
from pathlib import Path
import xml.etree.ElementTree as ET

import numpy as np

from . import scene as S

GEOM_TYPES = {'plane': S.PLANE, 'sphere': S.SPHERE, 'capsule': S.CAPSULE, 'ellipsoid': S.ELLIPSOID,
              'cylinder': S.CYLINDER, 'box': S.BOX, 'mesh': S.MESH}
JOINT_TYPES = {'free': S.FREE, 'ball': S.BALL, 'slide': S.SLIDE, 'hinge': S.HINGE}

# MuJoCo's built-in attribute values (the root of every default class)
BUILTIN = {
    'geom': dict(type='sphere', size='0 0 0', contype='1', conaffinity='1', condim='3', group='0',
                 priority='0', friction='1 0.005 0.0001', solmix='1', solref='0.02 1',
                 solimp='0.9 0.95 0.001 0.5 2', margin='0', gap='0', density='1000', pos='0 0 0'),
    'joint': dict(type='hinge', pos='0 0 0', axis='0 0 1', limited='auto', range='0 0', damping='0',
                  armature='0', stiffness='0', springref='0', frictionloss='0', margin='0',
                  solreflimit='0.02 1', solimplimit='0.9 0.95 0.001 0.5 2'),
    'site': dict(pos='0 0 0'),
}
ORIENTATION = ('quat', 'axisangle', 'euler', 'xyaxes', 'zaxis')
MINVAL = 1e-15


class MjcfError(ValueError):
    pass


@dataclass
class Compiler:
    angle: str = 'degree'
    eulerseq: str = 'xyz'
    inertiafromgeom: str = 'auto'
    inertiagrouprange: tuple = (0, 5)
    autolimits: bool = True
    boundmass: float = 0.0
    boundinertia: float = 0.0

    def update(self, el):
        if el is None:
            return self
        for key in ('angle', 'eulerseq', 'inertiafromgeom'):
            if key in el.attrib:
                setattr(self, key, el.get(key))
        if 'inertiagrouprange' in el.attrib:
            self.inertiagrouprange = tuple(int(x) for x in el.get('inertiagrouprange').split())
        if 'autolimits' in el.attrib:
            self.autolimits = el.get('autolimits') == 'true'
        for key in ('boundmass', 'boundinertia'):
            if key in el.attrib:
                setattr(self, key, float(el.get(key)))
        if self.angle not in ('degree', 'radian'):
            raise MjcfError('compiler angle must be degree or radian')
        return self


@dataclass
class XGeom:
    """A geom as written (attributes resolved against its default class), frame in its body."""
    name: str
    type: int
    size: tuple
    pos: np.ndarray
    quat: np.ndarray
    group: int
    contype: int
    conaffinity: int
    condim: int
    priority: int
    friction: tuple
    solref: tuple
    solimp: tuple
    solmix: float
    margin: float
    gap: float
    density: float
    mass: float | None
    mesh: str | None

    @property
    def visual(self):
        """Takes part in no collision (contype and conaffinity both 0)."""
        return self.contype == 0 and self.conaffinity == 0


@dataclass
class XBody:
    name: str
    pos: np.ndarray
    quat: np.ndarray
    inertial: dict | None = None             # mass, pos, quat, inertia (principal) from <inertial>
    joints: list = field(default_factory=list)      # scene.Joint (pos/axis in the body frame)
    joint_names: list = field(default_factory=list)
    geoms: list = field(default_factory=list)       # XGeom
    sites: list = field(default_factory=list)       # scene.Site
    children: list = field(default_factory=list)    # XBody


# ------------------------------------------------------------------------------ small math
def _floats(text, n=None):
    v = [float(x) for x in str(text).split()]
    if n is not None and len(v) != n:
        raise MjcfError('expected %d numbers, got %r' % (n, text))
    return v


def _filled(text, default):
    """A real vector attribute, completed from MuJoCo's built-in value where it is still short."""
    v = [float(x) for x in str(text).split()]
    d = [float(x) for x in str(default).split()]
    if not 0 < len(v) <= len(d):
        raise MjcfError('expected up to %d numbers, got %r' % (len(d), text))
    return tuple(v + d[len(v):])


def qmul(a, b):
    return np.array(S._qmul(a, b))


def quat2mat(q):
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def mat2quat(R):
    """Unit quaternion (w first, w >= 0) of a rotation matrix (Shepperd's method)."""
    R = np.asarray(R, float)
    tr = np.trace(R)
    if tr > 0:
        s = math.sqrt(tr + 1.0) * 2
        q = [0.25 * s, (R[2, 1] - R[1, 2]) / s, (R[0, 2] - R[2, 0]) / s, (R[1, 0] - R[0, 1]) / s]
    elif R[0, 0] > R[1, 1] and R[0, 0] > R[2, 2]:
        s = math.sqrt(1.0 + R[0, 0] - R[1, 1] - R[2, 2]) * 2
        q = [(R[2, 1] - R[1, 2]) / s, 0.25 * s, (R[0, 1] + R[1, 0]) / s, (R[0, 2] + R[2, 0]) / s]
    elif R[1, 1] > R[2, 2]:
        s = math.sqrt(1.0 + R[1, 1] - R[0, 0] - R[2, 2]) * 2
        q = [(R[0, 2] - R[2, 0]) / s, (R[0, 1] + R[1, 0]) / s, 0.25 * s, (R[1, 2] + R[2, 1]) / s]
    else:
        s = math.sqrt(1.0 + R[2, 2] - R[0, 0] - R[1, 1]) * 2
        q = [(R[1, 0] - R[0, 1]) / s, (R[0, 2] + R[2, 0]) / s, (R[1, 2] + R[2, 1]) / s, 0.25 * s]
    q = np.array(q)
    q /= np.linalg.norm(q)
    return q if q[0] >= 0 else -q


def axis_quat(axis, angle):
    axis = np.asarray(axis, float)
    axis = axis / np.linalg.norm(axis)
    s = math.sin(angle / 2)
    return np.array([math.cos(angle / 2), *(axis * s)])


def orientation(attrs, compiler):
    """Unit quaternion of an element's orientation attributes (MuJoCo's frame alternatives)."""
    scale = math.pi / 180 if compiler.angle == 'degree' else 1.0
    if 'quat' in attrs:
        q = np.array(_floats(attrs['quat'], 4))
    elif 'axisangle' in attrs:
        v = _floats(attrs['axisangle'], 4)
        q = axis_quat(v[:3], v[3] * scale)
    elif 'euler' in attrs:
        seq = compiler.eulerseq
        if len(seq) != 3 or any(c not in 'xyzXYZ' for c in seq):
            raise MjcfError('eulerseq must be three of x, y, z, X, Y, Z')
        q = np.array([1.0, 0.0, 0.0, 0.0])
        for c, a in zip(seq, _floats(attrs['euler'], 3)):
            r = axis_quat(np.eye(3)['xyz'.index(c.lower())], a * scale)
            q = qmul(q, r) if c.islower() else qmul(r, q)   # lowercase: axes that move with the frame
    elif 'xyaxes' in attrs:
        v = np.array(_floats(attrs['xyaxes'], 6))
        x = v[:3] / np.linalg.norm(v[:3])
        y = v[3:] - x * np.dot(x, v[3:])
        y /= np.linalg.norm(y)
        q = mat2quat(np.column_stack([x, y, np.cross(x, y)]))
    elif 'zaxis' in attrs:
        z = np.array(_floats(attrs['zaxis'], 3))
        z /= np.linalg.norm(z)
        c = np.cross([0.0, 0.0, 1.0], z)
        s, cz = np.linalg.norm(c), z[2]
        q = np.array([1.0, 0.0, 0.0, 0.0]) if s < 1e-12 and cz > 0 else \
            np.array([0.0, 1.0, 0.0, 0.0]) if s < 1e-12 else axis_quat(c / s, math.atan2(s, cz))
    else:
        q = np.array([1.0, 0.0, 0.0, 0.0])
    n = np.linalg.norm(q)
    if n < MINVAL:
        raise MjcfError('zero quaternion')
    return q / n


# ------------------------------------------------------------------------------ mass properties
def geom_volume_inertia(g):
    """Volume and unit-density principal inertia of a primitive in its own frame (MuJoCo's rules;
    a capsule is a cylinder of length 2 size[1] with hemispherical caps)."""
    s = g.size
    if g.type == S.SPHERE:
        r = s[0]
        v = 4.0 / 3.0 * math.pi * r ** 3
        return v, np.full(3, 0.4 * v * r * r)
    if g.type == S.BOX:
        a, b, c = s
        v = 8.0 * a * b * c
        return v, v / 3.0 * np.array([b * b + c * c, a * a + c * c, a * a + b * b])
    if g.type == S.CAPSULE:
        r, h = s[0], 2.0 * s[1]
        vs, vc = 4.0 / 3.0 * math.pi * r ** 3, math.pi * r * r * h
        ixx = vc * (3 * r * r + h * h) / 12 + vs * (0.4 * r * r + h * h / 4 + 3 * h * r / 8)
        return vs + vc, np.array([ixx, ixx, vc * r * r / 2 + vs * 0.4 * r * r])
    if g.type == S.CYLINDER:
        r, h = s[0], 2.0 * s[1]
        v = math.pi * r * r * h
        ixx = v * (3 * r * r + h * h) / 12
        return v, np.array([ixx, ixx, v * r * r / 2])
    if g.type == S.ELLIPSOID:
        a, b, c = s
        v = 4.0 / 3.0 * math.pi * a * b * c
        return v, v / 5.0 * np.array([b * b + c * c, a * a + c * c, a * a + b * b])
    raise MjcfError('no volume for geom type %d' % g.type)


def geom_mass(g):
    """Mass and principal inertia (geom frame) of a geom: mass given, or density times volume."""
    vol, unit = geom_volume_inertia(g)
    if g.mass is not None:
        density = g.mass / vol if vol > MINVAL else 0.0
        return g.mass, unit * density
    return g.density * vol, unit * g.density


def inertia_from_geoms(geoms):
    """Body mass, centre of mass, principal inertia and principal frame of a set of geoms."""
    parts = [(g, *geom_mass(g)) for g in geoms]
    mass = sum(p[1] for p in parts)
    if mass < MINVAL:
        return 0.0, np.zeros(3), np.zeros(3), np.array([1.0, 0.0, 0.0, 0.0])
    com = sum(p[1] * p[0].pos for p in parts) / mass
    full = np.zeros((3, 3))
    for g, m, inertia in parts:
        R = quat2mat(g.quat)
        d = g.pos - com
        full += R @ np.diag(inertia) @ R.T + m * (np.dot(d, d) * np.eye(3) - np.outer(d, d))
    principal, frame = principal_axes(full)
    return mass, com, principal, frame


def principal_axes(full):
    """Eigen-decomposition of a symmetric inertia: values in decreasing order and the right-handed
    frame of their axes as a quaternion."""
    vals, vecs = np.linalg.eigh(0.5 * (full + full.T))
    order = np.argsort(vals)[::-1]
    vals, vecs = vals[order], vecs[:, order]
    if np.linalg.det(vecs) < 0:
        vecs[:, 2] = -vecs[:, 2]
    return np.maximum(vals, 0.0), mat2quat(vecs)


# ------------------------------------------------------------------------------ parsing
# real-vector attributes of which MJCF allows a prefix: missing trailing values keep the values the
# element or class inherits (from its class, or from MuJoCo's built-ins)
VECTORS = {'friction', 'solref', 'solimp', 'solreflimit', 'solimplimit', 'size'}


def _merge(base, new):
    out = dict(base)
    for k, v in new.items():
        if k in VECTORS and k in base:
            vals, inherited = str(v).split(), str(base[k]).split()
            if len(vals) < len(inherited):
                v = ' '.join(vals + inherited[len(vals):])
        out[k] = v
    return out


class _Defaults:
    """Default classes: class name -> {tag: attrs}; nested classes inherit their parent's."""

    def __init__(self):
        self.classes = {'main': {tag: dict(v) for tag, v in BUILTIN.items()}}

    def read(self, el, parent='main'):
        name = el.get('class', 'main' if parent == 'main' and 'class' not in el.attrib else None)
        if name is None:
            raise MjcfError('nested default without a class')
        if name != 'main' or parent != 'main':
            self.classes[name] = copy.deepcopy(self.classes[parent])
        # the class's own element defaults first, then its nested classes (MuJoCo's order: a nested
        # class inherits every value of its parent, wherever the parent's elements are written)
        for child in el:
            if child.tag in ('geom', 'joint', 'site'):
                cls = self.classes[name]
                cls[child.tag] = _merge(cls.get(child.tag, {}), child.attrib)
            elif child.tag in ('inertial', 'body'):
                raise MjcfError('defaults for <%s> are not supported' % child.tag)
        for child in el:
            if child.tag == 'default':
                self.read(child, name)

    def attrs(self, el, childclass):
        cls = el.get('class', childclass or 'main')
        if cls not in self.classes:
            raise MjcfError('unknown default class %r' % cls)
        out = dict(self.classes[cls].get(el.tag, {}))
        if any(k in el.attrib for k in ORIENTATION):       # the element's own orientation wins
            for k in ORIENTATION:
                out.pop(k, None)
        return _merge(out, el.attrib)


class Mjcf:
    """One parsed MJCF file: compiler settings, options and the world body tree."""

    def __init__(self, root, compiler=None, source=''):
        if root.tag != 'mujoco':
            raise MjcfError('root element must be <mujoco>')
        self.source = source
        self.model = root.get('model', '')
        # an explicit compiler (e.g. the one a composed scene is compiled with) overrides the file's
        self.compiler = compiler if compiler is not None else Compiler().update(root.find('compiler'))
        self.option = dict(root.find('option').attrib) if root.find('option') is not None else {}
        flag = root.find('option/flag')
        self.flags = dict(flag.attrib) if flag is not None else {}
        self.defaults = _Defaults()
        for d in root.findall('default'):
            self.defaults.read(d)
        wb = root.find('worldbody')
        self.world = XBody('world', np.zeros(3), np.array([1.0, 0.0, 0.0, 0.0]))
        if wb is not None:
            self._fill(self.world, wb, None)

    # -- elements
    def _geom(self, el, childclass):
        a = self.defaults.attrs(el, childclass)
        if 'fromto' in a:
            raise MjcfError('geom fromto is not supported')
        gtype = a['type']
        if gtype not in GEOM_TYPES:
            raise MjcfError('geom type %r is not supported' % gtype)
        size = _floats(a['size'])
        size = tuple((size + [0.0, 0.0, 0.0])[:3])
        return XGeom(name=a.get('name', ''), type=GEOM_TYPES[gtype], size=size,
                     pos=np.array(_floats(a['pos'], 3)), quat=orientation(a, self.compiler),
                     group=int(a['group']), contype=int(a['contype']), conaffinity=int(a['conaffinity']),
                     condim=int(a['condim']), priority=int(a['priority']),
                     friction=_filled(a['friction'], BUILTIN['geom']['friction']),
                     solref=_filled(a['solref'], BUILTIN['geom']['solref']),
                     solimp=_filled(a['solimp'], BUILTIN['geom']['solimp']),
                     solmix=float(a['solmix']), margin=float(a['margin']), gap=float(a['gap']),
                     density=float(a['density']), mass=float(a['mass']) if 'mass' in a else None,
                     mesh=a.get('mesh'))

    def _joint(self, el, childclass):
        if el.tag == 'freejoint':
            return S.Joint(S.FREE), el.get('name', '')
        a = self.defaults.attrs(el, childclass)
        jtype = a['type']
        if jtype not in JOINT_TYPES:
            raise MjcfError('joint type %r is not supported' % jtype)
        jt = JOINT_TYPES[jtype]
        rng = _floats(a['range'], 2)
        if jt in (S.HINGE, S.BALL) and self.compiler.angle == 'degree':
            rng = [x * math.pi / 180 for x in rng]
        lim = a['limited']
        if lim == 'auto':
            if not self.compiler.autolimits:
                raise MjcfError('limited="auto" needs compiler autolimits')
            limited = rng != [0.0, 0.0]          # a range given (element or class): limited
        else:
            limited = lim == 'true'
        if limited and rng[0] >= rng[1]:
            raise MjcfError('joint range must be increasing when limited')
        j = S.Joint(jt, axis=tuple(_floats(a['axis'], 3)), pos=tuple(_floats(a['pos'], 3)), limited=bool(limited),
                    range=tuple(rng), damping=float(a['damping']), armature=float(a['armature']),
                    stiffness=float(a['stiffness']), springref=float(a['springref']),
                    frictionloss=float(a['frictionloss']), margin=float(a['margin']),
                    solref=_filled(a['solreflimit'], BUILTIN['joint']['solreflimit']),
                    solimp=_filled(a['solimplimit'], BUILTIN['joint']['solimplimit']))
        return j, a.get('name', '')

    def _site(self, el, childclass):
        a = self.defaults.attrs(el, childclass)
        return S.Site(pos=tuple(_floats(a['pos'], 3)), quat=tuple(orientation(a, self.compiler)),
                      name=a.get('name', ''))

    def _inertial(self, el):
        a = el.attrib
        mass = float(a['mass'])
        pos = np.array(_floats(a.get('pos', '0 0 0'), 3))
        quat = orientation(a, self.compiler)
        if 'diaginertia' in a:
            inertia = np.array(_floats(a['diaginertia'], 3))
        elif 'fullinertia' in a:
            xx, yy, zz, xy, xz, yz = _floats(a['fullinertia'], 6)
            full = np.array([[xx, xy, xz], [xy, yy, yz], [xz, yz, zz]])
            inertia, frame = principal_axes(full)
            quat = qmul(quat, frame)
        else:
            raise MjcfError('<inertial> needs diaginertia or fullinertia')
        return dict(mass=mass, pos=pos, quat=quat, inertia=inertia)

    def _fill(self, body, el, childclass):
        for child in el:
            tag = child.tag
            if tag == 'body':
                cc = child.get('childclass', childclass)
                a = dict(child.attrib)
                xb = XBody(a.get('name', ''), np.array(_floats(a.get('pos', '0 0 0'), 3)),
                           orientation(a, self.compiler))
                self._fill(xb, child, cc)
                body.children.append(xb)
            elif tag == 'geom':
                body.geoms.append(self._geom(child, childclass))
            elif tag in ('joint', 'freejoint'):
                if body.name == 'world':
                    raise MjcfError('joints in the world body')
                j, name = self._joint(child, childclass)
                body.joints.append(j)
                body.joint_names.append(name)
            elif tag == 'site':
                body.sites.append(self._site(child, childclass))
            elif tag == 'inertial':
                body.inertial = self._inertial(child)
            elif tag in ('camera', 'light'):
                continue
            elif tag in ('include', 'frame', 'composite', 'flexcomp', 'replicate'):
                raise MjcfError('<%s> is not supported' % tag)


def load(source, *, compiler=None):
    """Parse an MJCF file (path) or string."""
    text = str(source)
    if text.lstrip().startswith('<'):
        return Mjcf(ET.fromstring(text), compiler)
    path = Path(source)
    return Mjcf(ET.parse(path).getroot(), compiler, source=str(path))


# ------------------------------------------------------------------------------ compile
def in_group_range(g, compiler):
    lo, hi = compiler.inertiagrouprange
    return lo <= g.group <= hi


def body_mass_properties(xb, compiler):
    """MuJoCo's body inertia rule: <inertial> unless inertiafromgeom is true (or auto and absent)."""
    use_geoms = compiler.inertiafromgeom == 'true' or (compiler.inertiafromgeom == 'auto' and xb.inertial is None)
    if not use_geoms:
        if xb.inertial is None:
            return 0.0, np.zeros(3), np.zeros(3), np.array([1.0, 0.0, 0.0, 0.0])
        i = xb.inertial
        return i['mass'], i['pos'], i['inertia'], i['quat']
    massive = [g for g in xb.geoms if in_group_range(g, compiler) and g.type != S.PLANE]
    for g in massive:
        if g.type == S.MESH:
            raise MjcfError('mesh geom %r carries mass but its mesh data is not available' % g.name)
    return inertia_from_geoms(massive)


def compile_bodies(xworld, compiler, *, keep_visual=False, prefix=''):
    """World body plus its subtree as scene.Body objects in DFS preorder (world first).

    Geoms that collide with nothing are dropped unless ``keep_visual``; a collision mesh raises."""
    out = []

    def convert(xb, parent):
        name = prefix + xb.name if xb.name else prefix + 'body%d' % len(out)
        if parent < 0:
            body = S.Body('world', -1)
        else:
            mass, ipos, inertia, iquat = body_mass_properties(xb, compiler)
            mass = max(mass, compiler.boundmass) if xb.joints or compiler.boundmass else mass
            inertia = np.maximum(inertia, compiler.boundinertia)
            body = S.Body(name, parent, pos=tuple(xb.pos), quat=tuple(xb.quat), mass=float(mass),
                          inertia=tuple(float(x) for x in inertia), ipos=tuple(float(x) for x in ipos),
                          iquat=tuple(float(x) for x in iquat))
        for g in xb.geoms:
            if g.visual and not keep_visual:
                continue
            if g.type == S.MESH:
                raise MjcfError('collision mesh %r: mesh data is not available' % g.name)
            if g.type in (S.CYLINDER, S.ELLIPSOID):
                raise MjcfError('collision geom %r: cylinder and ellipsoid collisions are not supported' % g.name)
            body.geoms.append(S.Geom(g.type, size=g.size, pos=tuple(g.pos), quat=tuple(g.quat), contype=g.contype,
                                     conaffinity=g.conaffinity, condim=g.condim, priority=g.priority,
                                     friction=g.friction, solref=g.solref, solimp=g.solimp, solmix=g.solmix,
                                     margin=g.margin, gap=g.gap))
        body.joints = list(xb.joints)
        body.sites = [S.Site(pos=s.pos, quat=s.quat, name=prefix + s.name if s.name else '') for s in xb.sites]
        index = len(out)
        out.append(body)
        for child in xb.children:
            convert(child, index)

    convert(xworld, -1)
    return out


def counts(xb, *, include_self=True):
    """(bodies, joints, geoms, sites, nq, nv) of a subtree as MuJoCo would count them (every geom,
    visual ones included)."""
    nq = nv = 0
    for j in xb.joints:
        nq += {S.FREE: 7, S.BALL: 4}.get(j.type, 1)
        nv += {S.FREE: 6, S.BALL: 3}.get(j.type, 1)
    c = [1 if include_self else 0, len(xb.joints), len(xb.geoms), len(xb.sites), nq, nv]
    for child in xb.children:
        c = [a + b for a, b in zip(c, counts(child))]
    return c
