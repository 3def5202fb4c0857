# CMake package for the in-tree build of libkunlunk200.so.0: the same package
# and target names a consumer of the reference uses (find_package(KunlunK200
# CONFIG) and KunlunK200::kunlunk200, reference CMakeLists.txt:175-184), here an
# IMPORTED shared library over kunlunk200_lib_amd/lib and the public headers in
# include/. Point a consumer at it with -DKunlunK200_DIR=<this directory>.
get_filename_component(_kunlunk200_pkg "${CMAKE_CURRENT_LIST_DIR}/.." ABSOLUTE)
get_filename_component(_kunlunk200_root "${_kunlunk200_pkg}/.." ABSOLUTE)
set(_kunlunk200_lib "${_kunlunk200_pkg}/lib/libkunlunk200.so.0")
if(NOT EXISTS "${_kunlunk200_lib}")
    set(KunlunK200_FOUND FALSE)
    set(KunlunK200_NOT_FOUND_MESSAGE "${_kunlunk200_lib} is not built (run make -C kunlunk200_lib_amd/csrc)")
    return()
endif()
if(NOT TARGET KunlunK200::kunlunk200)
    add_library(KunlunK200::kunlunk200 SHARED IMPORTED)
    set_target_properties(KunlunK200::kunlunk200 PROPERTIES
        IMPORTED_LOCATION "${_kunlunk200_lib}"
        IMPORTED_SONAME "libkunlunk200.so.0"
        INTERFACE_INCLUDE_DIRECTORIES "${_kunlunk200_root}/include"
        INTERFACE_COMPILE_FEATURES cxx_std_14)
endif()
set(KunlunK200_INCLUDE_DIRS "${_kunlunk200_root}/include")
set(KunlunK200_LIBRARIES KunlunK200::kunlunk200)
set(KunlunK200_FOUND TRUE)
unset(_kunlunk200_lib)
unset(_kunlunk200_pkg)
unset(_kunlunk200_root)
